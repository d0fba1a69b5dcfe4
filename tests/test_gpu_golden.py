"""The HIP path against the committed golden vectors, through the C ABI, with
the same bars as the parity tests (the expectation is the stored oracle output,
not a live recomputation)."""
import pytest
import torch

from oracle import elementwise as ew
from oracle.numerics import assert_fused_cancel, assert_rel, assert_ulp, bits_equal
from tests.golden.loader import load

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def golden():
    return load()


def test_elementwise(gpu, golden):
    from thintnpu_amd import capi
    G = golden
    x, y = G["ew_x"].to(gpu), G["ew_y"].to(gpu)
    for op, name in ((capi.ADD, "add"), (capi.SUB, "sub"), (capi.MUL, "mul"), (capi.DIV, "div")):
        assert_ulp(capi.binary(op, x, y).cpu(), G[f"ew_{name}"], 0, name)
    assert_ulp(capi.binary(capi.ADD, x, y, 2.0).cpu(), G["ew_add_alpha2"], 0, "add alpha")
    assert_ulp(capi.binary(capi.SUB, x, y, 2.0).cpu(), G["ew_sub_alpha2"], 0, "sub alpha")
    assert_ulp(capi.unary(capi.SIGMOID, x).cpu(), G["ew_sigmoid"], 2, "sigmoid")
    assert_ulp(capi.unary(capi.SILU, x).cpu(), G["ew_silu"], 2, "silu")
    assert_fused_cancel(capi.silu_add(x, y).cpu(), G["ew_silu_add"], ew.silu(G["ew_x"].float()), 2, 4, "silu_add")
    got = capi.affine_silu(G["aff_x"].to(gpu), G["aff_s"].to(gpu), G["aff_b"].to(gpu)).cpu()
    assert_ulp(got, G["aff_y"], 2, "affine_silu")


def test_movement(gpu, golden):
    from thintnpu_amd import capi
    G = golden
    got = capi.cat([G["cat_a"].to(gpu), G["cat_b"].to(gpu), G["cat_c"].to(gpu)], 1).cpu()
    assert bits_equal(got, G["cat_dim1"])
    assert bits_equal(capi.upsample2x_nc1hwc0(G["up_x"].to(gpu)).cpu(), G["up_y"])
    assert bits_equal(capi.upsample2x_nchw(G["upn_x"].to(gpu)).cpu(), G["upn_y"])
    got = capi.upsample_cat_nc1hwc0([G["up_x"].to(gpu), G["upcat_b"].to(gpu)], [True, False]).cpu()
    assert bits_equal(got, G["upcat_y"])
    assert bits_equal(capi.pack_nc1hwc0(G["pack_x"].to(gpu)).cpu(), G["pack_y"])
    assert bits_equal(capi.unpack_nc1hwc0(G["pack_y"].to(gpu), 20).cpu(), G["unpack_y"])


def test_softmax_and_dfl(gpu, golden):
    from thintnpu_amd import capi
    G = golden
    # stored CPU fp16 softmax: 1e-3 absolute (the reference's bar, verify_softmax.py:57)
    got = capi.softmax(G["sm_x"].to(gpu), 1).cpu()
    torch.testing.assert_close(got.float(), G["sm_last"].float(), rtol=0, atol=1e-3, equal_nan=True)
    got = capi.softmax(G["sm_x"].to(gpu), 1, True).cpu()
    torch.testing.assert_close(got, G["sm_last_h2f"], rtol=0, atol=1e-6, equal_nan=True)
    got = capi.softmax(G["smd_x"].to(gpu).transpose(1, 2), 1).cpu()
    torch.testing.assert_close(got.float(), G["smd_dim1"].float(), rtol=0, atol=1e-3, equal_nan=True)
    assert_rel(capi.dfl_expect(G["dfl_x"].to(gpu)).cpu(), G["dfl_f16"], 1e-3, "dfl f16")
    assert_rel(capi.dfl_expect(G["dfl_x"].to(gpu), torch.float32).cpu(), G["dfl_f32"], 1e-5, "dfl f32")


@pytest.mark.parametrize("agnostic", [False, True])
def test_selection(gpu, golden, agnostic):
    from thintnpu_amd import capi
    from tests.test_gpu_selection import STAGES
    G = golden
    out, stages = capi.detection_select(G["sel_x"].to(gpu), 20, agnostic, trace=True)
    assert bits_equal(out.cpu(), G[f"sel_{int(agnostic)}_output"])
    for mine, theirs in STAGES.items():
        got = stages[mine].cpu()
        want = G[f"sel_{int(agnostic)}_{theirs}"]
        assert got.shape == want.shape, (mine, got.shape, want.shape)
        assert bits_equal(got, want.to(got.dtype)), mine


def test_bmm(gpu, golden):
    from thintnpu_amd import capi
    G = golden
    qkv, p = G["bmm_qkv"].to(gpu), G["bmm_p"].to(gpu)
    assert bits_equal(capi.layout_bmm(qkv, qkv, True, False, False, 2, 0, 16, 16, 16).cpu(), G["bmm_qk"])
    assert bits_equal(capi.layout_bmm(qkv, p, False, True, True, 2, 32, 16).cpu(), G["bmm_vp"])
    assert bits_equal(capi.channel_select(qkv, 2, 32, 16).cpu(), G["bmm_sel"])
    assert bits_equal(capi.bmm(G["bmm_a"].to(gpu), G["bmm_b"].to(gpu)).cpu(), G["bmm_ab"])

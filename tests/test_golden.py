"""The oracle against the committed golden vectors (tests/golden/golden.npz).

Closed-form ops (add/sub/mul/div with alpha, the sequential-sum bmm), data
movement and selection must
reproduce the stored bits on any torch build.  Exp-based ops (sigmoid, SiLU,
fused chains, softmax, DFL) are bit-identical on the torch version and CPU ISA
the manifest records and within one fp16 ulp (fp32: 1e-6 relative) elsewhere,
since torch's vectorised exp may move an ulp across versions and ISAs."""
import pytest
import torch

from oracle import bmm as ob
from oracle import elementwise as ew
from oracle import movement as mv
from oracle import reductions as rd
from oracle import selection as sel
from oracle.numerics import assert_ulp, bits_equal
from tests.golden.loader import load
from tests.golden.make_golden import cpu_isa

G = load()
SAME_BUILD = G["manifest"]["torch"] == torch.__version__ and G["manifest"]["cpu_isa"] == cpu_isa()


def exp_based(got, name):
    if SAME_BUILD:
        assert bits_equal(got, G[name]), name
    elif got.dtype == torch.float16:
        assert_ulp(got, G[name], 1, name)
    else:
        torch.testing.assert_close(got, G[name], rtol=1e-6, atol=0, equal_nan=True)


@pytest.fixture(autouse=True)
def one_thread():
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(threads)


def test_manifest():
    m = G["manifest"]
    assert m["torch"] and m["cpu_isa"] and m["threads"] == 1


def test_binary_bits():
    x, y = G["ew_x"], G["ew_y"]
    for op, name in ((3, "add"), (0, "sub"), (1, "mul"), (2, "div")):
        assert bits_equal(ew.binary(op, x, y), G[f"ew_{name}"]), name
    assert bits_equal(ew.binary(3, x, y, 2.0), G["ew_add_alpha2"])
    assert bits_equal(ew.binary(0, x, y, 2.0), G["ew_sub_alpha2"])


def test_exp_based():
    x, y = G["ew_x"], G["ew_y"]
    exp_based(ew.sigmoid(x), "ew_sigmoid")
    exp_based(ew.silu(x), "ew_silu")
    exp_based(ew.silu_add(x, y), "ew_silu_add")
    exp_based(ew.affine_silu(G["aff_x"], G["aff_s"], G["aff_b"]), "aff_y")
    exp_based(rd.softmax(G["sm_x"], 1), "sm_last")
    exp_based(rd.softmax(G["sm_x"], 1, True), "sm_last_h2f")
    exp_based(rd.softmax(G["smd_x"].transpose(1, 2), 1), "smd_dim1")
    exp_based(rd.dfl_expect(G["dfl_x"], torch.float16), "dfl_f16")
    exp_based(rd.dfl_expect(G["dfl_x"], torch.float32), "dfl_f32")


def test_movement_bits():
    assert bits_equal(mv.cat([G["cat_a"], G["cat_b"], G["cat_c"]], 1), G["cat_dim1"])
    assert bits_equal(mv.upsample2x_blocked(G["up_x"]), G["up_y"])
    assert bits_equal(mv.upsample2x_nchw(G["upn_x"]), G["upn_y"])
    assert bits_equal(mv.upsample_cat_blocked([G["up_x"], G["upcat_b"]], [True, False]), G["upcat_y"])
    assert bits_equal(mv.pack_blocked(G["pack_x"]), G["pack_y"])
    assert bits_equal(mv.unpack_blocked(G["pack_y"], 20), G["unpack_y"])


@pytest.mark.parametrize("agnostic", [False, True])
def test_selection_bits(agnostic):
    ref = sel.select(G["sel_x"], 20, agnostic)
    for name in sel.TRACE_NAMES:
        assert bits_equal(ref[name], G[f"sel_{int(agnostic)}_{name}"]), name


def test_bmm_bits():
    qkv, p = G["bmm_qkv"], G["bmm_p"]
    assert bits_equal(ob.layout_bmm(qkv, qkv, True, False, False, 2, 0, 16, 16, 16), G["bmm_qk"])
    assert bits_equal(ob.layout_bmm(qkv, p, False, True, True, 2, 32, 16), G["bmm_vp"])
    assert bits_equal(ob.channel_select(qkv, 2, 32, 16), G["bmm_sel"])
    assert bits_equal(ob.bmm(G["bmm_a"], G["bmm_b"]), G["bmm_ab"])
    assert G["bmm_ab"].isinf().any() and not G["bmm_ab"].isnan().any()

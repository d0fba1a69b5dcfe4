"""The PrivateUse1 ("npu") drop-in surface on the GPU: aten registrations,
thin_backend / thin_native_flow / thin_blocked / thin_fused ops, and the
CapturedForward / FrozenGraph capture-replay contract -- restating the
reference's verify_ops.py, verify_graph.py, verify_aten.py, verify_all.py,
verify_cat_plan.py, verify_dfl_softmax.py and verify_selection_flow.py device
checks.  Values are compared with the same CPU oracle as the C-ABI tests."""
import math
import os
import threading
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from oracle import elementwise as ew
from oracle import movement as mv
from oracle import reductions as rd
from oracle import selection as sel
from oracle.numerics import assert_rel, assert_ulp, bits_equal
from tests.helpers import gen, normal16, random_bits16, specials16, to_blocked

ROOT = Path(__file__).resolve().parent.parent

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def npu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    import thin_backend
    thin_backend.load_flow_libraries()
    return torch.device("npu:0")


def close(a, b, tol):
    assert a.device.type == "npu"
    got = a.cpu()
    assert got.shape == b.shape and got.dtype == b.dtype
    if got.dtype == torch.float16:
        assert_ulp(got, b, tol)
    else:
        torch.testing.assert_close(got, b, rtol=1e-5, atol=1e-5, equal_nan=True)


def test_binary_views_and_cat(npu):
    """verify_ops.py:68-143 restated."""
    g = gen(42)
    with torch.inference_mode():
        for dtype in (torch.float32, torch.float16):
            for shape in ((1,), (7,), (2047,), (2049,), (65537,), (0,), (), (3, 5, 7)):
                a = (torch.rand(shape, generator=g) * 2 - 1).to(dtype)
                b = (torch.rand(shape, generator=g) + 0.5).to(dtype)
                x, y = a.to(npu), b.to(npu)
                for op in ("sub", "mul", "div", "add"):
                    close(getattr(torch, op)(x, y), getattr(torch, op)(a, b), 0)
            a = torch.rand(2, 5, 7, generator=g).to(dtype)
            b = (torch.rand(2, 5, 7, generator=g) + 0.5).to(dtype)
            close(torch.sub(a.to(npu).transpose(0, 2), b.to(npu).transpose(0, 2)),
                  torch.sub(a.transpose(0, 2), b.transpose(0, 2)), 0)
            close(torch.sub(a.to(npu), b.to(npu), alpha=2), torch.sub(a, b, alpha=2), 0)
            close(a.to(npu) * 0.5, a * 0.5, 0)
            close(a.to(npu) + 1.25, a + 1.25, 0)
            # cat / split aliasing
            for dim in (0, 1, 2, -1):
                shape_b = [3, 5, 7]
                shape_b[dim % 3] = 4
                p, q = torch.randn(3, 5, 7, generator=g).to(dtype), torch.randn(shape_b, generator=g).to(dtype)
                assert bits_equal(torch.cat((p.to(npu), q.to(npu), p.to(npu)), dim).cpu(), torch.cat((p, q, p), dim))
            x = a.to(npu)
            for dim in (0, 1, 2):
                parts = torch.split(x, 2, dim)
                for part, ref in zip(parts, torch.split(a, 2, dim)):
                    assert part.untyped_storage().data_ptr() == x.untyped_storage().data_ptr()
                    assert bits_equal(part.cpu(), ref)
                assert bits_equal(torch.cat(parts, dim).cpu(), a)
            empty = torch.empty(0, dtype=dtype).to(npu)
            assert bits_equal(torch.cat((empty, x, empty), 1).cpu(), a)
            # views keep metadata
            for view in (lambda t: t.view(10, 7), lambda t: t.transpose(0, 2), lambda t: t.unsqueeze(1),
                         lambda t: t.unsqueeze(0).expand(4, -1, -1, -1), lambda t: t.as_strided((2, 3), (21, 7), 1)):
                v, r = view(x), view(a)
                assert v.stride() == r.stride() and v.storage_offset() == r.storage_offset()
                assert bits_equal(v.cpu(), r)


def test_silu_chain_in_place(npu):
    """silu_ on strided parents and the C2f split -> silu_ -> add -> cat chain."""
    with torch.inference_mode():
        for dtype in (torch.float32, torch.float16):
            a = torch.linspace(-4, 4, 2 * 7 * 5 * 7).reshape(2, 7, 5, 7).to(dtype)
            x = a.to(npu)
            pointer = x.data_ptr()
            out = F.silu(x, inplace=True)
            assert out is x and x.data_ptr() == pointer
            close(out, F.silu(a), 2)
            for channels in (8, 7):
                a = (torch.randn(2, channels, 13, 11, generator=gen(channels)) * 0.5).to(dtype)
                x = a.to(npu)
                p, q = torch.split(x, [channels // 2, channels - channels // 2], 1)
                rp, rq = torch.split(a.clone(), [channels // 2, channels - channels // 2], 1)
                F.silu(q, inplace=True)
                F.silu(rq, inplace=True)
                z = torch.cat((p, torch.add(q, q)), 1)
                close(z, torch.cat((rp, torch.add(rq, rq)), 1), 2)


def test_aten_routes_and_rejects(npu):
    """verify_aten.py:119-147: inherited ops and 'thin aten' rejections."""
    with torch.inference_mode():
        a = torch.randn(1, 7, 5, 7, generator=gen(1))
        an = a.to(npu)
        close(torch.softmax(an, 1), torch.softmax(a, 1), 0)
        assert bits_equal(torch.cat(an.split([3, 4], 1), 1).cpu(), a)
        close(torch.sigmoid(an), torch.sigmoid(a), 0)
        close(F.silu(an), F.silu(a), 0)
        close(an + torch.ones(1, 7, 1, 1).to(npu), a + 1, 0)
        assert bits_equal(F.interpolate(an, scale_factor=2, mode="nearest").cpu(),
                          F.interpolate(a, scale_factor=2, mode="nearest"))
        assert bits_equal(torch.ops.aten.upsample_nearest2d.vec(an, None, [2.0, 2.0]).cpu(),
                          F.interpolate(a, scale_factor=2, mode="nearest"))
        assert torch.arange(8, device="npu").cpu().tolist() == list(range(8))
        assert torch.full((2, 3), 2.0, device="npu").cpu().eq(2).all()
        assert torch.zeros(4, device="npu").cpu().eq(0).all()
        assert torch.tensor(1.5).to("npu").item() == 1.5
        # aten max_pool2d k5/s1/p2 (aten_adapter.cpp:61-80): values, zero placeholder indices
        assert bits_equal(F.max_pool2d(an, 5, 1, 2).cpu(), F.max_pool2d(a, 5, 1, 2))
        values, indices = torch.ops.aten.max_pool2d_with_indices(a.half().to(npu), [5, 5], [1, 1], [2, 2])
        assert bits_equal(values.cpu(), F.max_pool2d(a.half().float(), 5, 1, 2).half())
        assert indices.dtype == torch.int64 and not indices.cpu().any()
        assert bits_equal(torch.ops.thin_backend.maxpool2d(an).cpu(), F.max_pool2d(a, 5, 1, 2))
        for name, op in (("conv", lambda: F.conv2d(an, torch.randn(3, 7, 3, 3).to(npu))),
                         ("pool-k3", lambda: F.max_pool2d(an, 3, 1, 1)),
                         ("pool-s2", lambda: F.max_pool2d(an, 5, 2, 2)),
                         ("nearest-3x", lambda: F.interpolate(an, scale_factor=3, mode="nearest"))):
            with pytest.raises(RuntimeError, match="thin aten"):
                op()
        # aten::bmm is the sequential-fp32 fp16 contraction (bmm_flow.cpp:357-359)
        with pytest.raises(RuntimeError, match="FP16 rank-3"):
            torch.bmm(an[0], an[0])


def test_thin_backend_namespace(npu):
    """verify_all.py:59-126: thin_backend.add (fp32), sigmoid, upsample, Meta."""
    with torch.inference_mode():
        for size in (5000, 65537, 1, 2049, 0):
            a, b = torch.randn(size), torch.randn(size)
            close(torch.ops.thin_backend.add(a.to(npu), b.to(npu)), a + b, 0)
        for dtype in (torch.float32, torch.float16):
            for size in (1, 5000, 65537):
                x = torch.linspace(-8, 8, size, dtype=dtype)
                close(torch.ops.thin_backend.sigmoid(x.to(npu)), torch.sigmoid(x), 2)
            for shape in ((1, 2, 5, 7), (2, 3, 13, 11), (1, 64, 40, 40)):
                x = torch.randn(shape).to(dtype)
                assert bits_equal(torch.ops.thin_backend.upsample_nearest2d(x.to(npu)).cpu(),
                                  F.interpolate(x, scale_factor=2, mode="nearest"))
        for op, args in (("add", (torch.empty(5, device="meta"), torch.empty(5, device="meta"))),
                         ("sigmoid", (torch.empty(7, device="meta"),)),
                         ("upsample_nearest2d", (torch.empty(1, 16, 8, 8, device="meta"),))):
            assert getattr(torch.ops.thin_backend, op)(*args).device.type == "meta"
            for key in ("PrivateUse1", "AutogradPrivateUse1", "Meta"):
                assert torch._C._dispatch_has_kernel_for_dispatch_key("thin_backend::" + op, key)


def expression(x):
    return torch.sigmoid((x + x) * 0.5)


def test_graph_contract(npu):
    """verify_graph.py:14-69 restated."""
    from thin_backend.graph import CapturedForward
    with torch.inference_mode():
        x = torch.linspace(-2, 2, 2048).to(npu)
        graph = CapturedForward(expression, x)
        expected = expression(x).cpu()
        for _ in range(5):
            assert torch.equal(graph.replay().cpu(), expected)
        other = torch.linspace(1, 3, 2048).to(npu)
        assert torch.equal(graph(other).cpu(), expression(other).cpu())
        with pytest.raises(ValueError):
            graph(torch.empty(32, device="npu"))
        errors = []

        def wrong_thread():
            for call in (graph.replay, lambda: graph(x)):
                try:
                    call()
                except RuntimeError as error:
                    errors.append(str(error))
        t = threading.Thread(target=wrong_thread)
        t.start()
        t.join()
        assert len(errors) == 2 and all("creating thread/stream" in e for e in errors)
        second = CapturedForward(expression, x)
        retained = graph.outputs
        graph.close()
        graph.close()
        assert torch.equal(retained.cpu(), expression(other).cpu())
        assert torch.equal(second.replay().cpu(), expected)
        second.close()
        with pytest.raises(RuntimeError, match="Device-to-host"):
            CapturedForward(lambda value: value.cpu(), x)
        graph = CapturedForward(expression, x)
        retained = graph.outputs
        del graph
        assert torch.equal(retained.cpu(), expected)


def test_frozen_graph(npu):
    from blocked_graph import FrozenGraph

    class Pilot:
        calls = 0

        def validate(self):
            Pilot.calls += 1

    pilot = Pilot()
    with torch.inference_mode():
        x = torch.linspace(-2, 2, 4096).half().to(npu)
        g = FrozenGraph(pilot, expression, x)
        assert torch.equal(g.replay().cpu(), expression(x).cpu())
        y = torch.linspace(0, 1, 4096).half().to(npu)
        assert torch.equal(g(y).cpu(), expression(y).cpu())
        assert Pilot.calls == 3
        # the reference's surface: .graph is the CapturedForward, and a replay
        # made through it is validated too
        from thin_backend.graph import CapturedForward
        assert isinstance(g.graph, CapturedForward) and g.outputs is g.graph.outputs
        assert torch.equal(g.graph.replay().cpu(), expression(y).cpu())
        assert Pilot.calls == 4
        g.close()


def test_replays_enqueue_and_stay_ordered(npu):
    """RuntimeGraph.replay only enqueues (backend.cpp:89-93 in the reference):
    back-to-back replays of several captured forwards, then one read, equal the
    eager results; an eager op right after a replay on the same thread reads
    the replay's outputs; a changed input between replays is honoured."""
    from thin_backend.graph import CapturedForward
    with torch.inference_mode():
        xs = [normal16((2, 8, 20, 20, 16), 900 + i).to(npu) for i in range(4)]
        chain = lambda v: torch.cat([F.silu(v), v + v], dim=1)  # noqa: E731
        graphs = [CapturedForward(chain, x) for x in xs]
        eager = [chain(x).cpu() for x in xs]
        for _ in range(3):
            for g in graphs:
                g.replay()
        outs = [g.outputs.clone() for g in graphs]  # eager copies queued behind the replays
        for got, want in zip(outs, eager):
            assert bits_equal(got.cpu(), want)
        # an eager op consuming a replay's output without any synchronize
        for k in range(5):
            y = graphs[k % 4].replay()
            z = torch.mul(y, 0.5)
            assert bits_equal(z.cpu(), ew.binary_scalar(1, eager[k % 4], 0.5))  # op 1: mul
        # new inputs between queued replays
        for k in range(3):
            v = normal16((2, 8, 20, 20, 16), 950 + k).to(npu)
            out = graphs[1](v)
            assert bits_equal(out.cpu(), chain(v).cpu())
        assert all(g.graph.direct() for g in graphs)  # three kernels: dispatched directly
        for g in graphs:
            g.close()


def test_replay_dispatch_forms(npu):
    """Short kernel chains replay by direct dispatch of the recorded kernels,
    longer ones and recordings holding a copy node through hipGraphLaunch;
    every form equals the eager result on every replay, with eager work
    between the replays."""
    from thin_backend.graph import CapturedForward
    with torch.inference_mode():
        x = normal16((1, 4, 16, 16, 16), 960).to(npu)
        host = normal16((1, 4, 16, 16, 16), 961)

        def one(v):
            return torch.sigmoid(v)

        def four(v):
            return torch.cat([F.silu(v), (v + v) * 0.5], dim=1)

        def long(v):
            y = v
            for _ in range(6):
                y = F.silu(y) + v
            return y

        def with_upload(v):
            c = host.to(npu)  # a host-to-device copy node in the recording
            return F.silu(v) + c

        for fn, direct in ((one, True), (four, True), (long, False), (with_upload, False)):
            g = CapturedForward(fn, x)
            assert g.graph.direct() == direct, fn.__name__
            want = fn(x).cpu()
            for k in range(4):
                assert bits_equal(g.replay().cpu(), want), (fn.__name__, k)
                torch.sigmoid(x)  # eager work between replays
            other = normal16((1, 4, 16, 16, 16), 962 + k).to(npu)
            assert bits_equal(g(other).cpu(), fn(other).cpu()), fn.__name__
            g.close()


def test_runtime_graph_phases(npu):
    """thin_backend::RuntimeGraph refuses calls out of phase (empty ->
    recording -> executable -> closed) and stays usable for what is legal."""
    with torch.inference_mode():
        x = torch.linspace(-1, 1, 1024).to(npu)
        g = torch.classes.thin_backend.RuntimeGraph()
        with pytest.raises(RuntimeError, match="nothing to replay"):
            g.replay()
        with pytest.raises(RuntimeError, match="not recording"):
            g.end()
        g.begin()
        with pytest.raises(RuntimeError, match="records exactly once"):
            g.begin()
        y = torch.sigmoid(x)
        g.end()
        with pytest.raises(RuntimeError, match="records exactly once"):
            g.begin()
        g.replay()
        eager = torch.sigmoid(x).cpu()
        assert torch.equal(y.cpu(), eager)
        g.close()
        g.close()
        with pytest.raises(RuntimeError, match="closed"):
            g.replay()
        # a graph closed while recording discards the recording
        h = torch.classes.thin_backend.RuntimeGraph()
        h.begin()
        torch.sigmoid(x)
        h.close()
        assert torch.equal(torch.sigmoid(x).cpu(), eager)


def test_cross_thread_free_and_reuse(npu):
    """A block released by one host thread while another thread's stream
    could still read it must not be handed out again under that read.  Thread
    B computes sigmoid of a tensor that only B holds, then drops it; thread A
    at once allocates blocks of the same size on its own stream and
    overwrites them.  B's result must equal the oracle.  Eager ops finish
    before they return, as the reference's do (backend.cpp:46)."""
    x = random_bits16((1 << 24,), 88)          # 32 MB: a launch long enough to overlap
    with torch.inference_mode():
        expect = torch.sigmoid(x.to(npu)).cpu()  # the same kernel, one thread
        assert_ulp(expect, ew.sigmoid(x), 2)
        held = [x.to(npu)]                     # allocated on this thread's stream
        done = threading.Event()
        result = {}

        def reader():
            t = held.pop()
            y = torch.sigmoid(t)
            del t                              # the only reference: the block is released here
            result["y"] = y
            done.set()

        b = threading.Thread(target=reader)
        b.start()
        done.wait(60)
        junk = [torch.empty(1 << 24, dtype=torch.float16, device=npu).fill_(7.0) for _ in range(3)]
        b.join()
        assert "y" in result
        assert bits_equal(result["y"].cpu(), expect)
        assert all(bool((j.cpu() == 7.0).all()) for j in junk)


def test_async_mode_is_single_threaded(npu, tmp_path):
    """THIN_ASYNC=1 leaves eager ops asynchronous for one host thread; a
    second thread that touches the device raises instead of racing."""
    import subprocess
    import sys
    script = tmp_path / "async_probe.py"
    script.write_text(
        "import sys, threading, torch\n"
        f"sys.path.insert(0, {str(ROOT)!r})\n"
        "import thin_backend\n"
        "x = torch.linspace(-1, 1, 4096).to('npu')\n"
        "assert torch.equal((x + x).cpu(), x.cpu() + x.cpu())\n"
        "err = []\n"
        "def other():\n"
        "    try:\n"
        "        torch.sigmoid(x)\n"
        "    except RuntimeError as e:\n"
        "        err.append(str(e))\n"
        "t = threading.Thread(target=other); t.start(); t.join()\n"
        "assert err and 'THIN_ASYNC=1' in err[0], err\n"
        "print('async-probe-ok')\n")
    env = dict(os.environ, THIN_ASYNC="1")
    out = subprocess.run([sys.executable, str(script)], env=env, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and "async-probe-ok" in out.stdout, out.stderr[-2000:]


def test_cat_plan_capture_changed_input(npu):
    """verify_cat_plan.py:42-50: split -> cat captured, replayed with new inputs."""
    from thin_backend.graph import CapturedForward
    with torch.inference_mode():
        for dtype in (torch.float16, torch.float32):
            for count in (2, 6, 9, 17):
                x = torch.randn(1, count * 2, 20, 20, 16, generator=gen(count)).to(dtype)
                graph = CapturedForward(lambda v: torch.cat(v.split(2, 1), 1), x.to(npu))
                for scale in (1, -0.75, 0.5):
                    changed = x * scale
                    assert bits_equal(graph(changed.to(npu)).cpu(), changed)
                graph.close()


def test_scalar_operand_rounded_to_tensor_dtype(npu):
    """A 0-d CPU operand is converted to the tensor's dtype before the op, as
    the reference converts it (ops.cpp:466-467): C2PSA's q * key_dim**-0.5
    (whole_blocked.py:97) multiplies by the fp16 value of 1/sqrt(32).  The
    input draws enough values that PyTorch CPU's fp32-scalar rule gives
    different bits on some of them, so the check tells the rules apart."""
    x = torch.cat([random_bits16((200_000,), 77), specials16()])
    scale = 32 ** -0.5
    with torch.inference_mode():
        d = x.to(npu)
        for op, name in ((1, "mul"), (2, "div"), (3, "add"), (0, "sub")):
            got = getattr(torch, name)(d, scale).cpu()
            assert bits_equal(got, ew.binary_scalar_rounded(op, x, scale)), name
            if name in ("add", "sub"):
                continue
            got_first = getattr(torch, name)(torch.tensor(scale, dtype=torch.float64), d).cpu()
            assert bits_equal(got_first, ew.binary_scalar_rounded(op, x, scale, True)), name + " first"
        assert bits_equal((d * scale).cpu(), ew.binary_scalar_rounded(1, x, scale))
        assert not bits_equal((d * scale).cpu(), ew.binary_scalar(1, x, scale))


def test_strided_binary_eager_equals_capture(npu):
    """verify_strided_binary.py / verify_narrow_binary.py: eager == capture bitwise."""
    from thin_backend.graph import CapturedForward
    with torch.inference_mode():
        full = torch.randn(1, 3, 44, 76, 16, generator=gen(2931)).half().to(npu)
        grid = torch.randn(44, 76, 2, generator=gen(5)).half().to(npu)
        scalar = torch.tensor(2, dtype=torch.float16).to(npu)
        cases = [(full[..., :2], scalar), (full[..., 2:4], grid), (full[:, :1, ..., :2], full[..., :1]),
                 (full[..., 1:9], scalar)]
        for x, y in cases:
            for op in ("add", "sub", "mul", "div"):
                run = lambda _=None, x=x, y=y, op=op: getattr(torch, op)(x, y)
                eager = run().cpu()
                ref = getattr(torch, op)(x.cpu(), y.cpu())
                assert_ulp(eager, ref, 0)
                graph = CapturedForward(run, x)
                assert bits_equal(graph.replay().cpu(), eager)
                graph.close()


def test_dfl_softmax_capture(npu):
    """verify_dfl_softmax.py:25-52: the [B,16,4,A] DFL view via aten::_softmax,
    eager within tolerance and capture bitwise x3."""
    from thin_backend.graph import CapturedForward
    with torch.inference_mode():
        for width in (80, 8400):
            cpu = (torch.randn(2, 4, 16, width, generator=gen(width)) * 3).half()
            view = lambda t: t.transpose(1, 2)
            forward = lambda value: torch.ops.aten._softmax.default(view(value), 1, False)
            dev = cpu.to(npu)
            eager = forward(dev).cpu()
            assert_rel(eager, rd.softmax_rounded(view(cpu), 1), 1e-3, f"dfl {width}")
            graph = CapturedForward(forward, dev)
            for _ in range(3):
                assert bits_equal(graph.replay().cpu(), eager)
            graph.close()


def test_flow_ops(npu):
    """thin_native_flow.upsample / pack_input, thin_blocked.pack / unpack."""
    with torch.inference_mode():
        for c1, h, w, n in ((16, 20, 20, 1), (2, 13, 17, 1), (8, 40, 40, 3)):
            bits = random_bits16((n, c1, h, w, 16), c1 + h)
            assert bits_equal(torch.ops.thin_native_flow.upsample(bits.to(npu)).cpu(), mv.upsample2x_blocked(bits))
        x = random_bits16((1, 3, 32, 32), 3)
        assert bits_equal(torch.ops.thin_native_flow.pack_input(x.to(npu)).cpu(), mv.pack_blocked(x))
        x = random_bits16((2, 64, 20, 20), 4)
        y = torch.ops.thin_blocked.pack(x.to(npu))
        assert bits_equal(y.cpu(), mv.pack_blocked(x))
        assert bits_equal(torch.ops.thin_blocked.unpack(y).cpu(), x)
        xm = normal16((2, 64, 20, 20), 5)
        ym = torch.ops.thin_blocked.pack(xm.to(npu))
        assert bits_equal(torch.ops.thin_native_flow.maxpool(ym, 5).cpu(), mv.maxpool_blocked(mv.pack_blocked(xm), 5))
        with pytest.raises(RuntimeError, match="odd"):
            torch.ops.thin_native_flow.maxpool(ym, 4)
        # the SPPF block's three pools and concat as one op (cv2's input)
        assert bits_equal(torch.ops.thin_fused.sppf(ym).cpu(), mv.sppf_blocked(mv.pack_blocked(xm), 5, 3))
        pools = [ym]
        for _ in range(3):
            pools.append(torch.ops.thin_native_flow.maxpool(pools[-1], 5))
        assert bits_equal(torch.ops.thin_fused.sppf(ym, 5, 3).cpu(), torch.cat(pools, 1).cpu())
        with pytest.raises(RuntimeError, match="repeats"):
            torch.ops.thin_fused.sppf(ym, 5, 0)


def test_fused_ops(npu):
    with torch.inference_mode():
        x = to_blocked(normal16((2, 64, 40, 40), 1))
        y = to_blocked(normal16((2, 64, 40, 40), 2))
        got = torch.ops.thin_fused.silu_add(x.to(npu), y.to(npu)).cpu()
        assert ulp_ok(got, ew.silu_add(x, y))
        s = to_blocked((torch.rand(1, 64, 1, 1, generator=gen(3)) + 0.5).half())
        b = to_blocked((torch.randn(1, 64, 1, 1, generator=gen(4)) * 0.1).half())
        assert_ulp(torch.ops.thin_fused.affine_silu(x.to(npu), s.to(npu), b.to(npu)).cpu(), ew.affine_silu(x, s, b), 2)
        up = to_blocked(normal16((2, 64, 20, 20), 5))
        assert bits_equal(torch.ops.thin_fused.upsample_cat([up.to(npu), x.to(npu)], [1, 0]).cpu(),
                          mv.upsample_cat_blocked([up, x], [True, False]))
        logits = normal16((2, 64, 8400), 6, std=3.0)
        assert_rel(torch.ops.thin_fused.dfl_expect(logits.to(npu)).cpu(), rd.dfl_expect(logits, torch.float32), 1e-3)


def ulp_ok(got, ref):
    from oracle.numerics import ulp_report
    rep = ulp_report(got, ref)
    return rep["nan_match"] and rep["exact"] > 0.999 * rep["finite"]


def test_detection_select_eager_and_capture(npu):
    """verify_selection_flow.py:229-265: production == trace output, eager ==
    capture bitwise, changed-input replay bitwise, stages vs the oracle."""
    from tests.selection_fixtures import c5_selection_input
    with torch.inference_mode():
        x = c5_selection_input()
        base = x.transpose(1, 2).contiguous()
        dev = base.to(npu)
        view = lambda t: t.transpose(1, 2)
        out = torch.ops.thin_native_flow.detection_select(view(dev), 300, False)
        ref = sel.select(x, 300, False)
        assert bits_equal(out.cpu(), ref["output"])
        trace = torch.ops.thin_native_flow.detection_select_trace(view(dev), 300, False)
        assert len(trace) == 8 and bits_equal(trace[0].cpu(), ref["output"])
        for got, name in zip(trace[1:], sel.TRACE_NAMES[1:]):
            assert bits_equal(got.cpu(), ref[name].to(got.dtype)), name
        graph = torch.classes.thin_backend.RuntimeGraph()
        graph.begin()
        captured = torch.ops.thin_native_flow.detection_select(view(dev), 300, False)
        graph.end()
        graph.replay()
        assert bits_equal(captured.cpu(), out.cpu())
        changed = -base
        dev.copy_(changed.to(npu))
        changed_eager = torch.ops.thin_native_flow.detection_select(view(dev), 300, False).cpu()
        assert bits_equal(changed_eager, sel.select(view(changed), 300, False)["output"])
        graph.replay()
        assert bits_equal(captured.cpu(), changed_eager)
        graph.close()


def test_region_contract_guards_frozen_graph(npu):
    """RegionContract as FrozenGraph's pilot: replays while the region is
    frozen, ValueError once a parameter changes (blocked_graph.py:4-23,
    region_contract.py:5-28)."""
    import torch.nn as nn
    from blocked_graph import FrozenGraph
    from region_contract import RegionContract

    class Scale(nn.Module):
        def __init__(self):
            super().__init__()
            self.register_buffer("s", torch.full((1, 4, 1, 1, 16), 0.5, dtype=torch.float16).to(npu))

        def forward(self, x):
            return F.silu(torch.mul(x, self.s))

    with torch.no_grad():
        m = nn.Sequential(Scale()).eval()
        contract = RegionContract((m,))
        x = normal16((1, 4, 8, 8, 16), 3).to(npu)
        g = FrozenGraph(contract, m, x)
        assert bits_equal(g.replay().cpu(), m(x).cpu())
        m[0].s.copy_(m[0].s * 2)
        with pytest.raises(ValueError, match="version"):
            g.replay()
        g.close()
    with pytest.raises(ValueError, match="Expected fixed FP16 NPU"):
        RegionContract((nn.Linear(2, 2),))


def test_aten_trace_and_process_hygiene(npu, capfd, monkeypatch):
    """THIN_ATEN_TRACE=1 logs each aten -> thin route (aten_adapter.cpp:25-29);
    the process maps the native HIP libraries and spawns no children
    (verify_ops.py:36-50)."""
    import os
    x = torch.linspace(-3, 3, 4096).half().to(npu)
    monkeypatch.setenv("THIN_ATEN_TRACE", "1")
    torch.sigmoid(x)
    F.silu(x)
    torch.ops.aten.upsample_nearest2d.vec(x.view(1, 4, 32, 32), None, [2.0, 2.0])
    err = capfd.readouterr().err
    for route in ("aten::sigmoid -> thin_unary(SIGMOID)", "aten::silu -> thin_unary(SILU)",
                  "aten::upsample_nearest2d -> thin_upsample2x_nchw"):
        assert f"THIN_ATEN {route} device=npu:0" in err
    monkeypatch.delenv("THIN_ATEN_TRACE")
    torch.sigmoid(x)
    assert "THIN_ATEN" not in capfd.readouterr().err
    maps = open("/proc/self/maps").read()
    assert "libthin_hip.so" in maps and "libthin_backend.so" in maps
    def parent(pid):
        try:
            return int(open(f"/proc/{pid}/stat").read().rsplit(") ", 1)[1].split()[1])
        except (OSError, IndexError, ValueError):
            return None
    assert [p for p in os.listdir("/proc") if p.isdigit() and parent(p) == os.getpid()] == []


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_materialize_cases(npu, dtype):
    """verify_materialize.py:15-74 restated: permute(0,2,1).contiguous() with
    capture and changed-input replay, sliced / strided / expanded views, the
    strided-concat grid and raw-bit transposes."""
    from thin_backend.graph import CapturedForward
    bits = lambda t: t.cpu().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)  # noqa: E731
    g = gen(913)
    with torch.inference_mode():
        for groups, channels, rows in ((1, 16, 16), (3, 16, 6400), (2, 32, 48), (4, 48, 400), (2, 7, 19),
                                       (1, 85, 96)):
            x = torch.randn(groups, channels, rows, generator=g).to(dtype)
            forward = lambda value: value.permute(0, 2, 1).contiguous()  # noqa: E731
            expected = forward(x)
            assert torch.equal(bits(forward(x.to(npu))), bits(expected))
            graph = CapturedForward(forward, x.to(npu))
            assert torch.equal(bits(graph.replay()), bits(expected))
            changed = (x * 0.5).to(npu)
            assert torch.equal(bits(graph(changed)), bits(forward(changed)))
            graph.close()
        for shape in ((3, 128, 16), (2, 19, 7), (1, 32, 85), (4, 48, 32)):
            x = torch.randn(shape, generator=g).to(dtype)
            xn = x.to(npu)
            for view in (lambda t: t[..., 2:4], lambda t: t[..., 4:], lambda t: t[:, ::2, ::2],
                         lambda t: t[:, :1].expand(-1, 31, -1)):
                assert torch.equal(bits(view(xn).contiguous()), bits(view(x).contiguous()))
        for rows in (1, 7, 127, 128, 129, 6400):
            for widths in ((2, 2, 12), (1, 7, 24), (3, 5, 8), (6, 10)):
                sources = [torch.randn(rows, w, generator=g).to(dtype) for w in widths]
                values = [s.to(npu) for s in sources]
                want = torch.cat(sources, -1)
                assert torch.equal(bits(torch.cat(values, -1)), bits(want))
                graph = CapturedForward(lambda _: torch.cat(values, -1), values[0])
                assert torch.equal(bits(graph.replay()), bits(want))
                graph.close()
        for mode, transform in (("sliced", lambda t: t[::3]), ("broadcast", lambda t: t[:1].expand(273, -1)),
                                ("offset", lambda t: t[:, 1:])):
            sources = [torch.randn(273, w + (mode == "offset"), generator=g).to(dtype) for w in (2, 2, 12)]
            values = [transform(s.to(npu)) for s in sources]
            assert torch.equal(bits(torch.cat(values, -1)), bits(torch.cat([transform(s) for s in sources], -1)))
    raw = random_bits16((3, 32, 48), 913)
    with torch.inference_mode():
        assert bits_equal(raw.to(npu).transpose(1, 2).contiguous().cpu(), raw.transpose(1, 2).contiguous())
        slices = [raw[..., :2].contiguous(), raw[..., 2:4].contiguous(), raw[..., 4:16].contiguous()]
        assert bits_equal(torch.cat([s.to(npu) for s in slices], -1).cpu(), torch.cat(slices, -1))


def test_decode_constants(npu):
    """verify_decode.py restated: arange / full / stack / broadcast add /
    scalar mul and div / unbind / _local_scalar_dense on npu (decode.cpp:6-34)."""
    with torch.inference_mode():
        cases = {
            "arange": lambda d: torch.arange(80, device=d, dtype=torch.float32),
            "arange_step": lambda d: torch.arange(-2, 10, 0.5, device=d, dtype=torch.float32),
            "full": lambda d: torch.full((8400, 1), 8.0, device=d),
            "stack": lambda d: torch.stack((torch.arange(80, device=d, dtype=torch.float32),
                                            torch.arange(80, device=d, dtype=torch.float32)), dim=-1),
            "broadcast_add": lambda d: torch.arange(80, device=d, dtype=torch.float32).view(1, 80)
            + torch.full((2, 1), 0.5, device=d),
            "scalar_mul": lambda d: torch.arange(80, device=d, dtype=torch.float32) * 8,
            "scalar_div": lambda d: torch.arange(80, device=d, dtype=torch.float32) / 2,
        }
        for name, call in cases.items():
            torch.testing.assert_close(call("npu").cpu(), call("cpu"), rtol=0, atol=0, msg=name)
        x = torch.arange(12, device="npu", dtype=torch.float32).view(3, 4)
        torch.testing.assert_close(torch.stack(torch.unbind(x)).cpu(), torch.arange(12, dtype=torch.float32).view(3, 4))
        assert torch.full((), 8.0, device="npu").item() == 8.0


def test_reference_permute_sites(npu):
    """The reference's .contiguous()-after-permute call sites on npu tensors --
    the anchor head [B,na*no,H,W] -> [B,na,H,W,no] (whole_blocked.py:76) and the
    NCHW <-> NC1HWC0 repacks around depthwise (model_optimization.py:14,17) --
    bit-exact; each is a batched 2-D transpose."""
    with torch.inference_mode():
        head = normal16((2, 3 * 85, 20, 20), 3)
        got = head.to(npu).view(2, 3, 85, 20, 20).permute(0, 1, 3, 4, 2).contiguous()
        assert bits_equal(got.cpu(), head.view(2, 3, 85, 20, 20).permute(0, 1, 3, 4, 2).contiguous())
        x = normal16((2, 64, 20, 24), 4)
        blocked = x.to(npu).contiguous().view(2, 4, 16, 20, 24).permute(0, 1, 3, 4, 2).contiguous()
        assert bits_equal(blocked.cpu(), x.view(2, 4, 16, 20, 24).permute(0, 1, 3, 4, 2).contiguous())
        back = blocked.permute(0, 1, 4, 2, 3).contiguous().view(2, 64, 20, 24)
        assert bits_equal(back.cpu(), x)


def test_fused_head_ops_capture(npu):
    """thin_fused.sppf and thin_fused.detect_decode under CapturedForward
    (graph.py:14-51): a replay equals eager bitwise, and a call with a new input
    (copied into the captured one) gives the oracle's result for it."""
    from thin_backend.graph import CapturedForward
    with torch.inference_mode():
        x = to_blocked(normal16((2, 256, 20, 20), 21)).to(npu)
        graph = CapturedForward(lambda v: torch.ops.thin_fused.sppf(v), x)
        assert bits_equal(graph.replay().cpu(), torch.ops.thin_fused.sppf(x).cpu())
        x2 = to_blocked(normal16((2, 256, 20, 20), 22))
        assert bits_equal(graph(x2.to(npu)).cpu(), mv.sppf_blocked(x2, 5, 3))
        graph.close()
        shapes, strides = [8, 8, 4, 4], [8.0, 16.0]
        boxes, scores = normal16((1, 64, 80), 23, std=3.0), normal16((1, 3, 80), 24)
        sd = scores.to(npu)
        forward = lambda b: torch.ops.thin_fused.detect_decode(b, sd, shapes, strides)
        bd = boxes.to(npu)
        graph = CapturedForward(forward, bd)
        assert bits_equal(graph.replay().cpu(), forward(bd).cpu())
        boxes2 = normal16((1, 64, 80), 25, std=3.0)
        got = graph(boxes2.to(npu)).cpu()
        assert bits_equal(got, forward(boxes2.to(npu)).cpu())
        assert_ulp(got[:, 4:], ew.sigmoid(scores), 2)
        assert torch.isfinite(got).all() and got[:, :4].abs().sum() > 0
        graph.close()


def test_bmm_flow_eager_and_capture(npu):
    """verify_bmm_flow.py:14-40: torch.bmm on the device within 0.002 of torch's
    fp32 bmm and bit-equal to the sequential oracle; a RuntimeGraph replay
    equals eager, and after new operands are copied in, the replay equals a
    fresh eager call."""
    from oracle import bmm as ob
    g = gen(2026)
    with torch.inference_mode():
        for batch, m, k, n in ((4, 400, 32, 400), (4, 64, 400, 400), (2, 17, 9, 23), (3, 5, 37, 1031),
                               (1, 1, 1, 1)):
            for transposed in (False, True):
                a = (torch.randn(batch, k, m, generator=g).transpose(1, 2) if transposed
                     else torch.randn(batch, m, k, generator=g)).half()
                b = (torch.randn(batch, n, k, generator=g).transpose(1, 2) if transposed
                     else torch.randn(batch, k, n, generator=g)).half()
                left, right = a.to(npu), b.to(npu)
                actual = torch.bmm(left, right).cpu()
                torch.testing.assert_close(actual, torch.bmm(a.float(), b.float()).half(), rtol=0.002, atol=0.002)
                assert bits_equal(actual, ob.sequential_bmm(a, b))
                graph = torch.classes.thin_backend.RuntimeGraph()
                graph.begin()
                captured = torch.bmm(left, right)
                graph.end()
                graph.replay()
                assert bits_equal(captured.cpu(), actual)
                left.copy_((a * 0.5).to(npu))
                right.copy_((b * -0.25).to(npu))
                changed = torch.bmm(left, right).cpu()
                graph.replay()
                assert bits_equal(captured.cpu(), changed)
                graph.close()


def test_layout_bmm_and_channel_select_capture(npu):
    """verify_bmm_layout.py:86-106 through torch.ops.thin_native_flow: grouped
    q^T k, grouped v p^T with the blocked output and channel_select, each
    bit-equal to the oracle, to its capture and to a changed-input replay."""
    from oracle import bmm as ob
    ops = torch.ops.thin_native_flow

    def check(compute, expect, update):
        actual = compute().cpu().contiguous()
        assert bits_equal(actual, expect)
        graph = torch.classes.thin_backend.RuntimeGraph()
        graph.begin()
        captured = compute()
        graph.end()
        graph.replay()
        assert bits_equal(captured.cpu(), actual)
        update()
        changed = compute().cpu()
        graph.replay()
        assert bits_equal(captured.cpu(), changed)
        graph.close()

    with torch.no_grad():
        for heads, key, dim, tokens in ((4, 32, 64, 400), (4, 8, 16, 37), (8, 3, 6, 19)):
            group = 2 * key + dim
            logical = torch.randn(heads, group, tokens, generator=gen(heads + key)).half()
            source = logical.reshape(1, heads * group // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
            device = source.to(npu)
            qr, kr, vr = logical.split((key, key, dim), 1)
            check(lambda: ops.layout_bmm(device, device, True, False, False, heads, 0, key, key, key),
                  ob.sequential_bmm(qr.transpose(1, 2), kr), lambda: device.copy_((source * 0.5).to(npu)))
            device.copy_(source.to(npu))
            probability = torch.randn(heads, tokens, tokens, generator=gen(7)).half()
            pd = probability.to(npu)
            expect = ob.sequential_bmm(vr, probability.transpose(1, 2))
            expect = expect.reshape(1, heads * dim // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
            check(lambda: ops.layout_bmm(device, pd, False, True, True, heads, 2 * key, dim), expect,
                  lambda: (device.copy_((source * 0.5).to(npu)), pd.copy_((probability * 0.25).to(npu))))
            device.copy_(source.to(npu))
            expect = vr.reshape(1, heads * dim // 16, 16, tokens).permute(0, 1, 3, 2).contiguous()
            check(lambda: ops.channel_select(device, heads, 2 * key, dim), expect,
                  lambda: device.copy_((source * 0.5).to(npu)))
        # the unblocked result is the [.., :n] view of 16-column rows
        a = torch.randn(2, 5, 7, generator=gen(1)).half().to(npu)
        b = torch.randn(2, 7, 23, generator=gen(2)).half().to(npu)
        y = ops.bmm(a, b)
        assert y.shape == (2, 5, 23) and y.stride() == (5 * 32, 32, 1)
        with pytest.raises(RuntimeError, match="rank-3 operands"):
            ops.bmm(a.unsqueeze(0), b)


@pytest.mark.parametrize("prescale", [True, False])
@pytest.mark.parametrize("tokens", [400, 100])
def test_fused_attention_op(npu, prescale, tokens):
    """thin_native_flow.attention against the op chain of whole_blocked.py:91-103
    run op by op on the device, both orders of the scale: bit-equal.  400
    tokens run the fused kernel; 100 (not a multiple of 8) the chain itself,
    inside the op."""
    ops = torch.ops.thin_native_flow
    heads, key, dim = 4, 32, 64
    scale = key ** -0.5
    qkv_cpu = normal16((1, heads * (2 * key + dim) // 16, tokens, 16), 613 + tokens)
    with torch.inference_mode():
        qkv = qkv_cpu.to(npu)
        got = ops.attention(qkv, heads, key, dim, scale, prescale)
        if prescale:
            query = ops.channel_select(qkv, heads, 0, key) * scale
            scores = ops.layout_bmm(query, qkv, True, False, False, heads, 0, key, key, key)
        else:
            scores = ops.layout_bmm(qkv, qkv, True, False, False, heads, 0, key, key, key) * scale
        expect = ops.layout_bmm(qkv, scores.softmax(dim=-1), False, True, True, heads, 2 * key, dim)
    assert got.device.type == "npu" and got.shape == (1, heads * dim // 16, tokens, 16)
    assert bits_equal(got.cpu(), expect.cpu())
    with pytest.raises(RuntimeError, match="C0-aligned"):
        ops.attention(qkv, heads, key, 2, scale, prescale)


def test_attention_block_flow(npu):
    """The blocked attention forward of whole_blocked.py:91-110 (Q-prescaled
    order) on the device: channel_select, scale, grouped q^T k, row softmax,
    grouped v p^T with the blocked output, channel_select of v, add.  Each step
    is checked against the oracle applied to the device's own input to that
    step: exact everywhere except the softmax (1e-3 relative)."""
    from oracle import bmm as ob
    ops = torch.ops.thin_native_flow
    batch, num_heads, key_dim, head_dim, h, w = 1, 4, 32, 64, 20, 20
    tokens, heads = h * w, batch * num_heads
    scale = key_dim ** -0.5
    channels = num_heads * (2 * key_dim + head_dim)
    qkv_blocked = to_blocked(normal16((batch, channels, h, w), 31))          # [1, C1, h, w, 16]
    with torch.no_grad():
        qkv = qkv_blocked.to(npu).view(batch, -1, tokens, 16)
        selected = ops.channel_select(qkv, heads, 0, key_dim)
        query = selected * scale
        scores = ops.layout_bmm(query, qkv, True, False, False, heads, 0, key_dim, key_dim, key_dim)
        probability = scores.softmax(dim=-1)
        mixed = ops.layout_bmm(qkv, probability, False, True, True, heads, 2 * key_dim, head_dim)
        mixed = mixed.view(batch, num_heads * head_dim // 16, h, w, 16)
        position = ops.channel_select(qkv, heads, 2 * key_dim, head_dim).view(batch, -1, h, w, 16)
        out = mixed + position
    q_cpu = qkv_blocked.view(batch, -1, tokens, 16)
    assert bits_equal(selected.cpu(), ob.channel_select(q_cpu, heads, 0, key_dim))
    assert bits_equal(query.cpu(), ew.binary_scalar_rounded(1, selected.cpu(), scale))
    assert scores.shape == (heads, tokens, tokens)
    assert bits_equal(scores.cpu(), ob.layout_bmm(query.cpu(), q_cpu, True, False, False, heads, 0, key_dim,
                                                  key_dim, key_dim))
    assert_rel(probability.cpu(), rd.softmax(scores.cpu(), -1), 1e-3)
    expect = ob.layout_bmm(q_cpu, probability.cpu(), False, True, True, heads, 2 * key_dim, head_dim)
    assert bits_equal(mixed.cpu(), expect.view(batch, -1, h, w, 16))
    assert bits_equal(position.cpu(), ob.channel_select(q_cpu, heads, 2 * key_dim, head_dim).view(batch, -1, h, w, 16))
    assert bits_equal(out.cpu(), ew.binary(3, mixed.cpu(), position.cpu()))

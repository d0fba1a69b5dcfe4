"""Writes tests/golden/golden.npz: seeded small inputs of every op on the path
with the CPU oracle's outputs, plus a manifest of the torch / numpy versions
and CPU ISA they came from.

The reference commits no golden vectors (its fixtures are regenerated from
seeds, .gitignore:13-17); these pin the oracle against drift of torch's CPU
kernels (vectorised exp differs by an ulp across versions and ISAs) and give
the GPU tests a fixed expectation independent of the live oracle.  fp16
tensors are stored as their uint16 bits so NaN payloads survive.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import platform
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import bmm as ob  # noqa: E402
from oracle import elementwise as ew  # noqa: E402
from oracle import movement as mv  # noqa: E402
from oracle import reductions as rd  # noqa: E402
from oracle import selection as sel  # noqa: E402

OUT = Path(__file__).resolve().parent / "golden.npz"
SPECIALS = [0.0, -0.0, float("inf"), -float("inf"), float("nan"), 65504.0, -65504.0, 2 ** -24, -2 ** -24,
            2 ** -14, 1.0, -1.0, 0.5, 11.0, -11.0, 17.5, -17.5]


def gen(seed):
    return torch.Generator().manual_seed(seed)


def store(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def blocked(x: torch.Tensor) -> torch.Tensor:
    n, c, h, w = x.shape
    return x.view(n, c // 16, 16, h, w).permute(0, 1, 3, 4, 2).contiguous()


def cpu_isa() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("flags"):
                flags = set(line.split(":", 1)[1].split())
                for isa in ("avx512f", "avx2", "sse4_2"):
                    if isa in flags:
                        return isa
    except OSError:
        pass
    return platform.machine()


def build() -> dict[str, np.ndarray]:
    torch.set_num_threads(1)
    g = {}
    # elementwise: a flat fp16 vector of normals plus every special value
    base = (torch.randn(4000, generator=gen(42)) * 4).half()
    specials = torch.tensor(SPECIALS, dtype=torch.float16)
    x = torch.cat((base, specials.repeat_interleave(len(SPECIALS)), specials.repeat(len(SPECIALS))))
    y = torch.cat((((torch.rand(4000, generator=gen(43)) + 0.5) * 3).half(),
                   specials.repeat(len(SPECIALS)), specials.repeat_interleave(len(SPECIALS))))
    g["ew_x"], g["ew_y"] = store(x), store(y)
    for op, name in ((3, "add"), (0, "sub"), (1, "mul"), (2, "div")):
        g[f"ew_{name}"] = store(ew.binary(op, x, y))
    g["ew_add_alpha2"] = store(ew.binary(3, x, y, 2.0))
    g["ew_sub_alpha2"] = store(ew.binary(0, x, y, 2.0))
    g["ew_sigmoid"] = store(ew.sigmoid(x))
    g["ew_silu"] = store(ew.silu(x))
    g["ew_silu_add"] = store(ew.silu_add(x, y))
    # affine + SiLU on NC1HWC0 with a per-channel scale and bias
    ax = blocked((torch.randn(2, 32, 6, 5, generator=gen(44)) * 2).half())
    s = blocked((torch.rand(1, 32, 1, 1, generator=gen(45)) + 0.5).half())
    b = blocked((torch.randn(1, 32, 1, 1, generator=gen(46)) * 0.1).half())
    g["aff_x"], g["aff_s"], g["aff_b"] = store(ax), store(s), store(b)
    g["aff_y"] = store(ew.affine_silu(ax, s, b))
    # movement on raw bit patterns (NaN payloads included)
    bits = lambda shape, seed: torch.randint(-32768, 32768, shape, generator=gen(seed),  # noqa: E731
                                             dtype=torch.int32).to(torch.int16).view(torch.float16)
    c0, c1, c2 = bits((2, 1, 3, 4, 16), 50), bits((2, 3, 3, 4, 16), 51), bits((2, 2, 3, 4, 16), 52)
    g["cat_a"], g["cat_b"], g["cat_c"] = store(c0), store(c1), store(c2)
    g["cat_dim1"] = store(mv.cat([c0, c1, c2], 1))
    up = bits((2, 2, 3, 5, 16), 53)
    g["up_x"], g["up_y"] = store(up), store(mv.upsample2x_blocked(up))
    nchw = bits((2, 3, 4, 5), 54)
    g["upn_x"], g["upn_y"] = store(nchw), store(mv.upsample2x_nchw(nchw))
    other = bits((2, 3, 6, 10, 16), 55)
    g["upcat_b"], g["upcat_y"] = store(other), store(mv.upsample_cat_blocked([up, other], [True, False]))
    pk = bits((2, 20, 5, 7), 56)
    g["pack_x"] = store(pk)
    g["pack_y"] = store(mv.pack_blocked(pk))
    g["unpack_y"] = store(mv.unpack_blocked(mv.pack_blocked(pk), 20))
    # softmax: last dim, an inner dim, half_to_float; DFL expectation
    sm = (torch.randn(7, 400, generator=gen(2718)) * 3).half()
    g["sm_x"], g["sm_last"] = store(sm), store(rd.softmax(sm, 1))
    g["sm_last_h2f"] = store(rd.softmax(sm, 1, True))
    dv = (torch.randn(2, 4, 16, 40, generator=gen(1928)) * 3).half()
    g["smd_x"] = store(dv)
    g["smd_dim1"] = store(rd.softmax(dv.transpose(1, 2), 1))
    dl = (torch.randn(2, 64, 48, generator=gen(4)) * 3).half()
    g["dfl_x"] = store(dl)
    g["dfl_f16"] = store(rd.dfl_expect(dl, torch.float16))
    g["dfl_f32"] = store(rd.dfl_expect(dl, torch.float32))
    # selection: boxes and sigmoid scores with ties and NaNs, every trace stage
    sx = torch.cat(((torch.randn(1, 200, 4, generator=gen(149)) * 50).half(),
                    torch.rand(1, 200, 10, generator=gen(150)).half()), -1)
    sx[0, 5:25, 4:] = sx[0, 4, 4:]          # tied anchors
    sx[0, 30, 7] = float("nan")
    sx[0, 31, 4:] = 0.0
    g["sel_x"] = store(sx)
    for agnostic in (False, True):
        ref = sel.select(sx, 20, agnostic)
        for name in sel.TRACE_NAMES:
            g[f"sel_{int(agnostic)}_{name}"] = store(ref[name])
    # attention contractions: grouped q^T k, v p^T with the blocked output and
    # channel select over one [1,6,20,16] QKV tensor (2 heads of 16+16+16
    # channels), and a plain bmm whose large sums overflow to inf
    qkv = (torch.randn(1, 6, 20, 16, generator=gen(894)) * 2).half()
    prob = torch.rand(2, 20, 20, generator=gen(895)).half()
    g["bmm_qkv"], g["bmm_p"] = store(qkv), store(prob)
    g["bmm_qk"] = store(ob.layout_bmm(qkv, qkv, True, False, False, 2, 0, 16, 16, 16))
    g["bmm_vp"] = store(ob.layout_bmm(qkv, prob, False, True, True, 2, 32, 16))
    g["bmm_sel"] = store(ob.channel_select(qkv, 2, 32, 16))
    ma = (torch.randn(3, 7, 40, generator=gen(896)) * 100).half()
    mb = (torch.randn(3, 40, 9, generator=gen(897)) * 100).half()
    g["bmm_a"], g["bmm_b"], g["bmm_ab"] = store(ma), store(mb), store(ob.bmm(ma, mb))
    return g


def manifest() -> dict:
    return {"torch": torch.__version__, "numpy": np.__version__, "cpu_isa": cpu_isa(),
            "threads": 1, "python": platform.python_version()}


if __name__ == "__main__":
    data = build()
    data["manifest"] = np.frombuffer(json.dumps(manifest()).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")

#!/usr/bin/env python3
"""Benchmark of the FP16 blocked-layout tensor path on one MI355X.

One *step* = the per-channel broadcast affine + SiLU workload y = SiLU(x*s + b)
over NC1HWC0 fp16 tensors at the three YOLOv8s neck shapes (C,H,W) in
{(128,80,80), (256,40,40), (512,20,20)} with N=32, each run on the full tensor
and on the C2f half-split narrowed view x[:, C/2:] -- six launches of the
fused kernel.  ``value`` = algorithmic bytes (each input read once, each output
written once, 2 B per fp16) of a step / step time, in GB/s, with inputs resident
in HBM and buffer sets rotated (>= 1.25 GB) so the 256 MB Infinity Cache cannot
serve them.  Consecutive steps are replayed from HIP graphs holding 8 steps each
(every step on its own rotated set); exactly --steps steps are timed.

Also reported (``ops``): per-op / per-chain µs and GB/s at N=1 (cache-resident
and rotated) and N=32 for every op built, each beside the reference's CPU path
(the stock PyTorch CPU op sequence) timed on the host cores, the roofline of
the dominant kernel, and the CPU path of the step itself (``cpu_baseline``).
Only rank 0 prints: one compact JSON line on stdout (the headline, roofline and
CPU baseline); progress and the per-op rows (one JSON object per line) go to
stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

os.environ.setdefault("TORCH_DEVICE_BACKEND_AUTOLOAD", "0")
ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

METRIC = "HBM GB/s (% of peak) + µs/op, YOLOv8s fp16 eltwise/softmax, N=1 & N=32"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 1280 << 20  # distinct buffer bytes a rotated row cycles through: 5x the 256 MB Infinity Cache
# (with 2.8x, three sets of the C3 upsample->cat at N=32, rows still came
# partly from the cache: 35.7 against 49.4 us with six sets)
GRAPH_STEPS = 8           # bench steps recorded in one HIP graph
C2_SHAPES = [(128, 80, 80), (256, 40, 40), (512, 20, 20)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ inputs

def gen(seed):
    return torch.Generator().manual_seed(seed)


def blocked_normal(n, c, h, w, seed, dev, std=1.0, mean=0.0):
    """NC1HWC0 fp16 [n, c/16, h, w, 16] with N(mean, std) values, made on the GPU
    from a seeded GPU generator (the parity tests use CPU-seeded inputs; timing
    only needs the right shapes and value ranges)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn((n, c // 16, h, w, 16), generator=g, device=dev) * std + mean).half()


def c2_set(n, c, h, w, dev, seed):
    x = blocked_normal(n, c, h, w, seed, dev)
    g = torch.Generator(device=dev).manual_seed(seed + 7)
    s = (torch.rand((1, c // 16, 1, 1, 16), generator=g, device=dev) + 0.5).half()
    b = (torch.randn((1, c // 16, 1, 1, 16), generator=g, device=dev) * 0.1).half()
    y = torch.empty_like(x)
    return x, s, b, y


# ------------------------------------------------------------------ timing

def capture(fn):
    """Record fn()'s launches (enqueued on torch's current stream, which the
    C-ABI wrappers use) into a HIP graph via torch's graph capture."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def time_launches(launch, sets, iters, rounds=5):
    """Median over `rounds` of (event elapsed / iters) for one replay of a HIP
    graph holding `iters` back-to-back launches cycling through `sets` (graph
    replay removes host launch cost, so this is device time per launch).  HIP
    events are recorded on the stream that replays the graph.  Seconds."""
    for i in range(min(len(sets), 3)):
        launch(sets[i])
    torch.cuda.synchronize()
    g = capture(lambda: [launch(sets[i % len(sets)]) for i in range(iters)])
    stream = torch.cuda.current_stream()
    g.replay()
    torch.cuda.synchronize()
    res = []
    for _ in range(rounds):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g.replay()
        stop.record(stream)
        stop.synchronize()
        res.append(start.elapsed_time(stop) / 1e3 / iters)
    del g
    return statistics.median(res)


# rocprofv3 --pmc readings of the dominant kernel, affine_silu_flat_kernel at
# N=32 (128,80,80): memory requests the L2 sent to HBM per dispatch, by size
# (TCC_EA0_RDREQ_32B/_64B/_128B, TCC_EA0_WRREQ and TCC_EA0_WRREQ_64B, summed over
# the L2 channels, median over 123 dispatches) from
# `bench.py --profile dominant --iters 20` (profiles/affine_silu_flat_n32_128x80x80_pmc.md).
# Every request is counted once at its size, so bytes = sum(size x count)
# without any calibration; write requests that are not 64-byte are 32-byte.
DOMINANT_REQUESTS = {"RDREQ_32B": 0, "RDREQ_64B": 320, "RDREQ_128B": 409632, "WRREQ": 819200, "WRREQ_64B": 819200}


def dominant_traffic():
    """HBM bytes per launch of the dominant kernel from its request counters."""
    r = DOMINANT_REQUESTS
    read = 32 * r["RDREQ_32B"] + 64 * r["RDREQ_64B"] + 128 * r["RDREQ_128B"]
    write = 64 * r["WRREQ_64B"] + 32 * (r["WRREQ"] - r["WRREQ_64B"])
    return read + write


def rotation_count(bytes_per_set):
    return max(2, math.ceil(ROTATE_BYTES / max(1, bytes_per_set)))


# ------------------------------------------------------------------ ops

def op_affine_silu(capi, dev, n, c, h, w, narrowed, rotate=True):
    """Returns (launch, sets, algorithmic bytes)."""
    c1 = c // 16
    per = n * c1 * h * w * 16 * 2
    frac = 0.5 if narrowed else 1.0
    algo = int(per * frac * 2 + 2 * c1 * 16 * 2 * frac)
    nsets = rotation_count(per * 2) if rotate else 1
    sets = [c2_set(n, c, h, w, dev, 11 + i) for i in range(nsets)]

    def launch(st):
        x, s, b, y = st
        if narrowed:
            capi.affine_silu(x[:, c1 // 2:], s[:, c1 // 2:], b[:, c1 // 2:], out=y[:, c1 // 2:])
        else:
            capi.affine_silu(x, s, b, out=y)
    return launch, sets, algo


def op_silu_add(capi, dev, n, rotate=True):
    per = n * 4 * 160 * 160 * 16 * 2
    nsets = rotation_count(per * 3) if rotate else 1
    sets = [(blocked_normal(n, 64, 160, 160, 21 + i, dev), blocked_normal(n, 64, 160, 160, 51 + i, dev),
             torch.empty((n, 4, 160, 160, 16), dtype=torch.float16, device=dev)) for i in range(nsets)]

    def launch(st):
        capi.silu_add(st[0], st[1], out=st[2])
    return launch, sets, per * 3


def rotated(make, per_set_bytes, rotate):
    n = rotation_count(per_set_bytes) if rotate else 1
    return [make(i) for i in range(n)]


def op_pack(capi, dev, n, rotate=True):
    """C1 repack NCHW [n,64,160,160] -> NC1HWC0 [n,4,160,160,16]."""
    per = n * 64 * 160 * 160 * 2
    g = torch.Generator(device=dev).manual_seed(5)
    sets = rotated(lambda i: (torch.randn((n, 64, 160, 160), generator=g, device=dev).half(),
                              torch.empty((n, 4, 160, 160, 16), dtype=torch.float16, device=dev)), per * 2, rotate)
    return (lambda st: capi.pack_nc1hwc0(st[0], out=st[1])), sets, per * 2


def op_cat_c2f(capi, dev, n, rotate=True):
    """C3 C2f cat of 4 chunks [n,64,80,80] (two halves of one [n,128,80,80])."""
    chunk = n * 4 * 80 * 80 * 16 * 2

    def make(i):
        parent = blocked_normal(n, 128, 80, 80, 30 + i, dev)
        return (parent, blocked_normal(n, 64, 80, 80, 60 + i, dev), blocked_normal(n, 64, 80, 80, 90 + i, dev),
                torch.empty((n, 16, 80, 80, 16), dtype=torch.float16, device=dev))
    sets = rotated(make, chunk * 8, rotate)

    def launch(st):
        a, b = st[0][:, :4], st[0][:, 4:]
        capi.cat([a, b, st[1], st[2]], 1, out=st[3])
    return launch, sets, chunk * 8


def op_upsample(capi, dev, n, rotate=True):
    """C3 nearest 2x [n,256,40,40] -> [n,256,80,80] in NC1HWC0."""
    src = n * 16 * 40 * 40 * 16 * 2
    sets = rotated(lambda i: (blocked_normal(n, 256, 40, 40, 120 + i, dev),
                              torch.empty((n, 16, 80, 80, 16), dtype=torch.float16, device=dev)), src * 5, rotate)
    return (lambda st: capi.upsample2x_nc1hwc0(st[0], out=st[1])), sets, src * 5


def op_upsample_cat(capi, dev, n, rotate=True):
    """C3 fused: cat(up2x([n,256,40,40]), [n,128,80,80]) -> [n,384,80,80]."""
    up = n * 16 * 40 * 40 * 16 * 2
    other = n * 8 * 80 * 80 * 16 * 2
    algo = up + other + n * 24 * 80 * 80 * 16 * 2
    sets = rotated(lambda i: (blocked_normal(n, 256, 40, 40, 150 + i, dev), blocked_normal(n, 128, 80, 80, 180 + i, dev),
                              torch.empty((n, 24, 80, 80, 16), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.upsample_cat_nc1hwc0([st[0], st[1]], [True, False], out=st[2])), sets, algo


def op_dfl(capi, dev, n, rotate=True):
    """C4 DFL [n,64,8400] -> [n,4,8400] fp16."""
    algo = n * (64 * 8400 * 2 + 4 * 8400 * 2)
    g = torch.Generator(device=dev).manual_seed(4)
    sets = rotated(lambda i: ((torch.randn((n, 64, 8400), generator=g, device=dev) * 3).half(),
                              torch.empty((n, 4, 8400), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.dfl_expect(st[0], out=st[1])), sets, algo


def op_sigmoid(capi, dev, n, rotate=True):
    """C4 class sigmoid [n,80,8400]."""
    algo = n * 80 * 8400 * 2 * 2
    g = torch.Generator(device=dev).manual_seed(14)
    sets = rotated(lambda i: ((torch.randn((n, 80, 8400), generator=g, device=dev) * 2 - 4).half(),
                              torch.empty((n, 80, 8400), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.unary(capi.SIGMOID, st[0], out=st[1])), sets, algo


def op_bcast_binary(capi, dev, n, c, h, w, op, narrowed, rotate=True):
    """What aten mul / add run on the device for an NC1HWC0 [n,C1,H,W,16]
    tensor and a per-channel [1,C1,1,1,16] operand (the unfused scale and
    shift of a convolution's output, ops.cpp:464-497 of the reference): one
    thin_binary launch over the broadcast view into a fresh contiguous output,
    on the full tensor or the C2f half x[:, C1/2:]."""
    c1 = c // 16
    full = n * c1 * h * w * 16 * 2
    part = full // 2 if narrowed else full
    algo = 2 * part + (c1 // 2 if narrowed else c1) * 16 * 2

    def make(i):
        x = blocked_normal(n, c, h, w, 400 + i, dev)
        g = torch.Generator(device=dev).manual_seed(500 + i)
        s = (torch.rand((1, c1, 1, 1, 16), generator=g, device=dev) + 0.5).half()
        if narrowed:
            x, s = x[:, c1 // 2:], s[:, c1 // 2:]
        return x, s, torch.empty(x.shape, dtype=torch.float16, device=dev)
    sets = rotated(make, full + part, rotate)
    return (lambda st: capi.binary(op, st[0], st[1], out=st[2])), sets, algo


def op_c1_unary_binary(capi, dev, n, which, rotate=True):
    """C1 as separate aten ops: SiLU of [n,64,160,160] NC1HWC0, or the add of
    two such tensors (the residual), each one launch."""
    per = n * 4 * 160 * 160 * 16 * 2
    if which == "silu":
        sets = rotated(lambda i: (blocked_normal(n, 64, 160, 160, 600 + i, dev),
                                  torch.empty((n, 4, 160, 160, 16), dtype=torch.float16, device=dev)), per * 2, rotate)
        return (lambda st: capi.unary(capi.SILU, st[0], out=st[1])), sets, per * 2
    sets = rotated(lambda i: (blocked_normal(n, 64, 160, 160, 620 + i, dev), blocked_normal(n, 64, 160, 160, 640 + i, dev),
                              torch.empty((n, 4, 160, 160, 16), dtype=torch.float16, device=dev)), per * 3, rotate)
    return (lambda st: capi.binary(capi.ADD, st[0], st[1], out=st[2])), sets, per * 3


C2F_CHAIN = (128, 80, 80)  # the C2f tensor the captured chain runs on


def c2f_chain(x):
    """The tail of a C2f block as a drop-in caller writes it: split the
    convolution's output in two, SiLU in place on one half, the residual add,
    and the concatenation (NC1HWC0 channel blocks, dim 1)."""
    a, b = x.split(x.shape[1] // 2, dim=1)
    torch.nn.functional.silu(b, inplace=True)
    return torch.cat([a, b, a + b], dim=1)


def c2f_chain_bytes(n):
    c, h, w = C2F_CHAIN
    half = n * (c // 32) * h * w * 16 * 2
    return 11 * half  # silu_ 2, add 3, cat 6 halves


def time_c2f_captured(n, replays, rounds=5, rotate=True):
    """Wall-clock seconds per CapturedForward replay of c2f_chain on the npu
    device (a HIP graph launched on the calling thread's stream; replays are
    asynchronous, so back-to-back replays measure the device time unless the
    graph is shorter than its host launch).  Buffers rotate over several
    captured forwards like the other rows."""
    import thin_backend  # noqa: F401  (the npu device)
    from thin_backend.graph import CapturedForward
    c, h, w = C2F_CHAIN
    npu = torch.device("npu:0")
    count = rotation_count(c2f_chain_bytes(n)) if rotate else 1
    graphs = []
    with torch.inference_mode():
        for i in range(count):
            x = torch.randn((n, c // 16, h, w, 16), generator=gen(700 + i)).half().to(npu)
            graphs.append(CapturedForward(c2f_chain, x))
        for gph in graphs:
            gph.replay()
        thin_backend.synchronize()
        res = []
        for _ in range(rounds):
            t0 = time.perf_counter()
            for k in range(replays):
                graphs[k % count].replay()
            thin_backend.synchronize()
            res.append((time.perf_counter() - t0) / replays)
        for gph in graphs:
            gph.close()
    return statistics.median(res)


def op_softmax(capi, dev, n, rotate=True):
    """C5 attention row softmax [n,4,400,400]."""
    algo = n * 4 * 400 * 400 * 2 * 2
    g = torch.Generator(device=dev).manual_seed(5)
    sets = rotated(lambda i: ((torch.randn((n, 4, 400, 400), generator=g, device=dev) * 2).half(),
                              torch.empty((n, 4, 400, 400), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.softmax(st[0], 3, out=st[1])), sets, algo


def op_maxpool(capi, dev, n, rotate=True):
    """SPPF max pool k5 on NC1HWC0 [n,256,20,20] (one of the three chained pools)."""
    algo = n * 16 * 20 * 20 * 16 * 2 * 2
    sets = rotated(lambda i: (blocked_normal(n, 256, 20, 20, 210 + i, dev),
                              torch.empty((n, 16, 20, 20, 16), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.maxpool_nc1hwc0(st[0], 5, out=st[1])), sets, algo


def op_dfl_softmax(capi, dev, n, rotate=True):
    """The DFL bin softmax as the reference's aten path computes it
    (softmax_host.cpp:29-50): softmax over dim 1 of x.view(n,4,16,A).transpose(1,2)
    for logits [n,64,8400], written to a contiguous [n,16,4,8400]."""
    a = 8400
    algo = n * 64 * a * 2 * 2
    g = torch.Generator(device=dev).manual_seed(9)
    sets = rotated(lambda i: ((torch.randn((n, 64, a), generator=g, device=dev) * 3).half(),
                              torch.empty((n, 16, 4, a), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.softmax(st[0].view(n, 4, 16, a).transpose(1, 2), 1, out=st[1])), sets, algo


def op_sppf(capi, dev, n, rotate=True):
    """SPPF pooling + concat on NC1HWC0 [n,256,20,20]: cat([x, p(x), p(p(x)),
    p(p(p(x)))], 1), p the k5 pool, in one pass (x read once, 4 slots written)."""
    algo = n * 16 * 20 * 20 * 16 * 2 * 5
    sets = rotated(lambda i: (blocked_normal(n, 256, 20, 20, 230 + i, dev),
                              torch.empty((n, 64, 20, 20, 16), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.sppf_nc1hwc0(st[0], 5, 3, out=st[1])), sets, algo


def op_decode(capi, dev, n, rotate=True):
    """Anchor-free head decode: DFL [n,64,8400] + sigmoid [n,80,8400] -> [n,84,8400]."""
    a = 8400
    algo = n * a * 2 * (64 + 80 + 84)
    g = torch.Generator(device=dev).manual_seed(6)
    sets = rotated(lambda i: ((torch.randn((n, 64, a), generator=g, device=dev) * 3).half(),
                              (torch.randn((n, 80, a), generator=g, device=dev) * 2 - 4).half(),
                              torch.empty((n, 84, a), dtype=torch.float16, device=dev)), algo, rotate)
    shapes, strides = [(80, 80), (40, 40), (20, 20)], [8.0, 16.0, 32.0]
    return (lambda st: capi.detect_decode(st[0], st[1], shapes, strides, out=st[2])), sets, algo


def op_decode_direct(capi, dev, n, rotate=True):
    """YOLO26 head decode (reg_max = 1, distances as given): [n,4,8400] +
    sigmoid [n,80,8400] -> [n,84,8400]."""
    a = 8400
    algo = n * a * 2 * (4 + 80 + 84)
    g = torch.Generator(device=dev).manual_seed(8)
    sets = rotated(lambda i: ((torch.rand((n, 4, a), generator=g, device=dev) * 20).half(),
                              (torch.randn((n, 80, a), generator=g, device=dev) * 2 - 4).half(),
                              torch.empty((n, 84, a), dtype=torch.float16, device=dev)), algo, rotate)
    shapes, strides = [(80, 80), (40, 40), (20, 20)], [8.0, 16.0, 32.0]
    return (lambda st: capi.detect_decode(st[0], st[1], shapes, strides, out=st[2])), sets, algo


def op_permute(capi, dev, n, rotate=True):
    """Materialize NCHW [n,64,80,80] as NHWC: x.permute(0,2,3,1).contiguous()."""
    algo = n * 64 * 80 * 80 * 2 * 2
    sets = rotated(lambda i: (torch.randn((n, 64, 80, 80), device=dev).half(),
                              torch.empty((n, 80, 80, 64), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.copy(st[0].permute(0, 2, 3, 1), st[1])), sets, algo


# C2PSA attention of YOLO26 at a 640x640 input: 4 heads, key 32, head 64, the
# 20x20 = 400 tokens of P5, over one N=1 blocked QKV tensor (N=1 only: head
# groups need an N=1 operand, as in the reference)
ATTN = (4, 32, 64, 400)


def attn_qkv(dev, seed):
    heads, key, dim, tokens = ATTN
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn((1, heads * (2 * key + dim) // 16, tokens, 16), generator=g, device=dev).half()


def op_attn_qk(capi, dev, n, rotate=True):
    """Attention scores per head, q^T k: [400,32] x [32,400] from the grouped
    blocked QKV (layout_bmm), [4,400,400] fp16 out; 41 MFLOP."""
    heads, key, dim, tokens = ATTN
    algo = heads * (2 * key * tokens + tokens * tokens) * 2
    sets = rotated(lambda i: (attn_qkv(dev, 300 + i),
                              torch.empty((heads, tokens, tokens), dtype=torch.float16, device=dev)), algo, rotate)
    return (lambda st: capi.layout_bmm(st[0], st[0], True, False, False, heads, 0, key, key, key, out=st[1])), \
        sets, algo


def op_attn_pv(capi, dev, n, rotate=True):
    """Attention mix per head, v p^T: [64,400] x [400,400] with the blocked
    output [1,16,400,16] (layout_bmm, grouped); 82 MFLOP."""
    heads, key, dim, tokens = ATTN
    algo = heads * (2 * dim * tokens + tokens * tokens) * 2
    g = torch.Generator(device=dev).manual_seed(11)
    sets = rotated(lambda i: (attn_qkv(dev, 310 + i),
                              torch.rand((heads, tokens, tokens), generator=g, device=dev).half(),
                              torch.empty((1, heads * dim // 16, tokens, 16), dtype=torch.float16, device=dev)),
                   algo, rotate)
    return (lambda st: capi.layout_bmm(st[0], st[1], False, True, True, heads, 2 * key, dim, out=st[2])), \
        sets, algo


def attn_fused_bytes():
    """qkv read once, mixed values written once."""
    heads, key, dim, tokens = ATTN
    return (heads * (2 * key + dim) + heads * dim) * tokens * 2


def op_attn_fused(capi, dev, n, prescale, rotate=True):
    """The whole attention chain of one C2PSA block in one launch
    (thin_attention): qkv [1,32,400,16] -> mixed values [1,16,400,16]; 123
    MFLOP, bit-equal to the chain below."""
    heads, key, dim, tokens = ATTN
    algo = attn_fused_bytes()
    scale = float(torch.tensor(key ** -0.5, dtype=torch.float64).half())
    sets = rotated(lambda i: (attn_qkv(dev, 330 + i),
                              torch.empty((1, heads * dim // 16, tokens, 16), dtype=torch.float16, device=dev)),
                   algo, rotate)
    return (lambda st: capi.attention(st[0], heads, key, dim, scale, prescale, out=st[1])), sets, algo


def op_attn_chain(capi, dev, n, prescale, rotate=True):
    """The same chain op by op, as attention_forward runs it: channel_select,
    mul, layout_bmm (q^T k), row softmax, layout_bmm (v p^T) -- five launches
    (four in the post-scale form, where the mul follows the product)."""
    heads, key, dim, tokens = ATTN
    algo = attn_fused_bytes()
    scale = float(torch.tensor(key ** -0.5, dtype=torch.float64).half())

    def buffers(i):
        return (attn_qkv(dev, 340 + i),
                torch.empty((1, heads * key // 16, tokens, 16), dtype=torch.float16, device=dev),
                torch.empty((1, heads * key // 16, tokens, 16), dtype=torch.float16, device=dev),
                torch.empty((heads, tokens, tokens), dtype=torch.float16, device=dev),
                torch.empty((heads, tokens, tokens), dtype=torch.float16, device=dev),
                torch.empty((heads, tokens, tokens), dtype=torch.float16, device=dev),
                torch.empty((1, heads * dim // 16, tokens, 16), dtype=torch.float16, device=dev))
    sets = rotated(buffers, algo, rotate)

    def run(st):
        qkv, sel, query, scores, scaled, prob, out = st
        if prescale:
            capi.channel_select(qkv, heads, 0, key, out=sel)
            capi.binary_scalar(capi.MUL, sel, scale, out=query)
            capi.layout_bmm(query, qkv, True, False, False, heads, 0, key, key, key, out=scores)
            capi.softmax(scores, 2, out=prob)
        else:
            capi.layout_bmm(qkv, qkv, True, False, False, heads, 0, key, key, key, out=scores)
            capi.binary_scalar(capi.MUL, scores, scale, out=scaled)
            capi.softmax(scaled, 2, out=prob)
        capi.layout_bmm(qkv, prob, False, True, True, heads, 2 * key, dim, out=out)
    return run, sets, algo


def op_attn_select(capi, dev, n, rotate=True):
    """channel_select of v (the position branch input): [1,16,400,16] out."""
    heads, key, dim, tokens = ATTN
    algo = heads * dim * tokens * 2 * 2
    sets = rotated(lambda i: (attn_qkv(dev, 320 + i),
                              torch.empty((1, heads * dim // 16, tokens, 16), dtype=torch.float16, device=dev)),
                   algo, rotate)
    return (lambda st: capi.channel_select(st[0], heads, 2 * key, dim, out=st[1])), sets, algo


def op_select(capi, dev, layout, rotate=False):
    """C5 NMS-free top-300 of [1,8400,84] (latency-bound: report us)."""
    from tests.selection_fixtures import c5_selection_input  # input generator, shared with the tests
    x = c5_selection_input()
    base = x.transpose(1, 2).contiguous() if layout == "transposed" else x.contiguous()
    d = base.to(dev)
    view = d.transpose(1, 2) if layout == "transposed" else d
    out = torch.empty((1, 300, 6), dtype=torch.float32, device=dev)
    ws = torch.empty(capi.detection_select_workspace(1, 8400, 80, 300, False), dtype=torch.uint8, device=dev)
    algo = 8400 * 84 * 2 + 300 * 6 * 4
    return (lambda st: capi.detection_select(view, 300, False, out=out, workspace=ws)), [None], algo


def op_rows(capi, dev):
    """(name, cfg, N, factory) for the per-op table."""
    rows = []
    for n in (1, 32):
        rows.append(("silu_add", "C1", n, lambda r, n=n: op_silu_add(capi, dev, n, r)))
        rows.append(("pack_nc1hwc0", "C1", n, lambda r, n=n: op_pack(capi, dev, n, r)))
    for n in (1, 32):
        for (c, h, w) in C2_SHAPES:
            for narrowed in (False, True):
                name = f"affine_silu{'_narrowed' if narrowed else ''}_{c}x{h}x{w}"
                rows.append((name, "C2", n, lambda r, n=n, c=c, h=h, w=w, nr=narrowed:
                             op_affine_silu(capi, dev, n, c, h, w, nr, r)))
    for n in (1, 32):
        for which in ("silu", "add"):
            rows.append((f"{which}_c1", "C1", n, lambda r, n=n, wh=which: op_c1_unary_binary(capi, dev, n, wh, r)))
    for (c, h, w) in C2_SHAPES:
        for opname, op in (("mul", capi.MUL), ("add", capi.ADD)):
            for narrowed in (False, True):
                name = f"aten_{opname}_bcast{'_narrowed' if narrowed else ''}_{c}x{h}x{w}"
                rows.append((name, "C2", 32, lambda r, c=c, h=h, w=w, op=op, nr=narrowed:
                             op_bcast_binary(capi, dev, 32, c, h, w, op, nr, r)))
    for n in (1, 32):
        rows.append(("cat_c2f_4x64", "C3", n, lambda r, n=n: op_cat_c2f(capi, dev, n, r)))
        rows.append(("upsample2x_256x40x40", "C3", n, lambda r, n=n: op_upsample(capi, dev, n, r)))
        rows.append(("upsample_cat_256+128", "C3", n, lambda r, n=n: op_upsample_cat(capi, dev, n, r)))
        rows.append(("dfl_expect_64x8400", "C4", n, lambda r, n=n: op_dfl(capi, dev, n, r)))
        rows.append(("sigmoid_80x8400", "C4", n, lambda r, n=n: op_sigmoid(capi, dev, n, r)))
        rows.append(("dfl_softmax_16x4x8400", "C4", n, lambda r, n=n: op_dfl_softmax(capi, dev, n, r)))
        rows.append(("softmax_4x400x400", "C5", n, lambda r, n=n: op_softmax(capi, dev, n, r)))
        rows.append(("maxpool_k5_256x20x20", "SPPF", n, lambda r, n=n: op_maxpool(capi, dev, n, r)))
        rows.append(("sppf_k5x3_cat_256x20x20", "SPPF", n, lambda r, n=n: op_sppf(capi, dev, n, r)))
        rows.append(("detect_decode_64+80x8400", "C4", n, lambda r, n=n: op_decode(capi, dev, n, r)))
        rows.append(("detect_decode_4+80x8400", "C5", n, lambda r, n=n: op_decode_direct(capi, dev, n, r)))
        rows.append(("permute_nchw_to_nhwc_64x80x80", "MAT", n, lambda r, n=n: op_permute(capi, dev, n, r)))
    rows.append(("attn_qk_4x32x400", "ATTN", 1, lambda r: op_attn_qk(capi, dev, 1, r)))
    rows.append(("attn_pv_4x64x400", "ATTN", 1, lambda r: op_attn_pv(capi, dev, 1, r)))
    rows.append(("channel_select_4x64x400", "ATTN", 1, lambda r: op_attn_select(capi, dev, 1, r)))
    for form in ("prescale", "postscale"):
        pre = form == "prescale"
        rows.append((f"attn_fused_{form}_4x32x64x400", "ATTN", 1,
                     lambda r, pre=pre: op_attn_fused(capi, dev, 1, pre, r)))
        rows.append((f"attn_chain_{form}_4x32x64x400", "ATTN", 1,
                     lambda r, pre=pre: op_attn_chain(capi, dev, 1, pre, r)))
    for layout in ("contiguous", "transposed"):
        rows.append((f"detection_select_{layout}", "C5", 1, lambda r, l=layout: op_select(capi, dev, l)))
    return rows


# ------------------------------------------------------------------ HBM size sweep

SWEEP_MB = (13, 26, 52, 105, 210, 315)
FLUSH_BYTES = 512 << 20


def sweep_mixes(capi, dev):
    """(name, read:write mix, factory(target algorithmic bytes) -> (launch,
    sets, algorithmic bytes)) for the HBM size sweep: plain streaming
    kernels of the library at several read:write mixes, plus the kernels
    judged against them (the dominant affine+SiLU, upsample->cat, DFL)."""
    h = torch.float16

    def dense(m, i):
        return torch.randn(m, generator=torch.Generator(device=dev).manual_seed(900 + i), device=dev).half()

    def copy(target):
        m = max(8, int(target) // 4 // 8 * 8)
        sets = rotated(lambda i: (dense(m, i), torch.empty(m, dtype=h, device=dev)), 4 * m, True)
        return (lambda st: capi.copy(st[0], st[1])), sets, 4 * m

    def add(target):
        m = max(8, int(target) // 6 // 8 * 8)
        sets = rotated(lambda i: (dense(m, i), dense(m, 50 + i), torch.empty(m, dtype=h, device=dev)), 6 * m, True)
        return (lambda st: capi.binary(capi.ADD, st[0], st[1], out=st[2])), sets, 6 * m

    def fill(target):
        m = max(8, int(target) // 2 // 8 * 8)
        sets = rotated(lambda i: (torch.empty(m, dtype=h, device=dev),), 2 * m, True)
        return (lambda st: capi.fill(st[0], 1.0)), sets, 2 * m

    def images(target, per_image):
        return max(1, round(target / per_image))

    return [
        ("copy", "1:1", copy),
        ("add", "2:1", add),
        ("fill", "0:1", fill),
        ("affine_silu_128x80x80", "1:1", lambda t: op_affine_silu(capi, dev, images(t, 3276800), 128, 80, 80,
                                                                   False, True)),
        ("upsample_cat_256+128", "1:2", lambda t: op_upsample_cat(capi, dev, images(t, 7372800), True)),
        ("dfl_expect_64x8400", "16:1", lambda t: op_dfl(capi, dev, images(t, 1142400), True)),
    ]


def fit_line(points):
    """Least-squares t = t0 + bytes / BW over (bytes, seconds) points:
    (t0 in us, BW in GB/s, largest relative residual)."""
    n = len(points)
    mx = sum(b for b, _ in points) / n
    my = sum(t for _, t in points) / n
    sxx = sum((b - mx) ** 2 for b, _ in points)
    slope = sum((b - mx) * (t - my) for b, t in points) / sxx
    t0 = my - slope * mx
    worst = max(abs(t0 + slope * b - t) / t for b, t in points)
    return t0 * 1e6, 1.0 / slope / 1e9, worst


def hbm_sweep(capi, dev, iters):
    """Rotated launches of each mix at SWEEP_MB sizes, the per-mix fit, and
    cold-cache times (a 512 MB fill before every launch, its own time taken
    off) for the N=32 kernels the fits judge."""
    fits = {}
    for name, mix, factory in sweep_mixes(capi, dev):
        points = []
        for mb in SWEEP_MB:
            launch, sets, algo = factory(mb * 1e6)
            t = time_launches(launch, sets, iters)
            points.append((algo, t))
            print(json.dumps({"sweep": name, "mix": mix, "bytes": algo, "us": round(t * 1e6, 3),
                              "GB/s": round(algo / t / 1e9, 1)}), flush=True)
            del sets
            torch.cuda.empty_cache()
        t0, bw, worst = fit_line(points)
        fits[name] = (t0, bw)
        print(json.dumps({"fit": name, "mix": mix, "t0_us": round(t0, 3), "GB/s": round(bw, 1),
                          "pct_peak": round(100 * bw / HBM_PEAK_GBS, 1), "max_rel_residual": round(worst, 4)}),
              flush=True)
    scratch = torch.empty(FLUSH_BYTES // 2, dtype=torch.float16, device=dev)
    fill_t = time_launches(lambda st: capi.fill(scratch, 0.0), [None], max(20, iters // 4))
    for name, factory in (("affine_silu_128x80x80", lambda: op_affine_silu(capi, dev, 32, 128, 80, 80, False, True)),
                          ("upsample_cat_256+128", lambda: op_upsample_cat(capi, dev, 32, True)),
                          ("dfl_expect_64x8400", lambda: op_dfl(capi, dev, 32, True))):
        launch, sets, algo = factory()

        def flushed(st, launch=launch):
            capi.fill(scratch, 0.0)
            launch(st)
        t = time_launches(flushed, sets, max(20, iters // 4)) - fill_t
        print(json.dumps({"flushed": name, "N": 32, "bytes": algo, "us": round(t * 1e6, 3),
                          "GB/s": round(algo / t / 1e9, 1), "fill_512MB_us": round(fill_t * 1e6, 3)}), flush=True)
        del sets
        torch.cuda.empty_cache()
    return fits


# ------------------------------------------------------------------ CPU baseline

def cpu_op(name, n):
    """(callable, algorithmic bytes) running the reference's CPU path of one op
    row -- the stock PyTorch CPU op sequence its tests compare against -- on
    seeded CPU tensors of the row's shape; None for rows without one."""
    import torch.nn.functional as F
    g = gen(7)
    h16 = lambda *shape: torch.randn(shape, generator=g).half()  # noqa: E731
    if name == "silu_add":
        x, y = h16(n, 4, 160, 160, 16), h16(n, 4, 160, 160, 16)
        return (lambda: y + F.silu(x)), n * 4 * 160 * 160 * 16 * 2 * 3
    if name in ("silu_c1", "add_c1"):
        x, y = h16(n, 4, 160, 160, 16), h16(n, 4, 160, 160, 16)
        return ((lambda: F.silu(x)), x.numel() * 4) if name == "silu_c1" else ((lambda: x + y), x.numel() * 6)
    if name.startswith("aten_"):
        c, h, w = (int(v) for v in name.rsplit("_", 1)[1].split("x"))
        c1 = c // 16
        x, sc = h16(n, c1, h, w, 16), h16(1, c1, 1, 1, 16).abs() + 0.5
        if "narrowed" in name:
            x, sc = x[:, c1 // 2:], sc[:, c1 // 2:]
        fn = (lambda: x * sc) if name.startswith("aten_mul") else (lambda: x + sc)
        return fn, x.numel() * 4
    if name == "c2f_chain_captured":
        c, h, w = C2F_CHAIN
        x = h16(n, c // 16, h, w, 16)
        return (lambda: c2f_chain(x)), c2f_chain_bytes(n)
    if name == "pack_nc1hwc0":
        x = h16(n, 64, 160, 160)
        return (lambda: x.view(n, 4, 16, 160, 160).permute(0, 1, 3, 4, 2).contiguous()), x.numel() * 4
    if name.startswith("affine_silu"):
        c, h, w = (int(v) for v in name.rsplit("_", 1)[1].split("x"))
        c1 = c // 16
        x, sc, b = h16(n, c1, h, w, 16), h16(1, c1, 1, 1, 16).abs() + 0.5, h16(1, c1, 1, 1, 16) * 0.1
        if "narrowed" in name:
            x, sc, b = x[:, c1 // 2:], sc[:, c1 // 2:], b[:, c1 // 2:]
        return (lambda: F.silu(torch.add(torch.mul(x, sc), b))), x.numel() * 4
    if name == "cat_c2f_4x64":
        parent, c, d = h16(n, 8, 80, 80, 16), h16(n, 4, 80, 80, 16), h16(n, 4, 80, 80, 16)
        return (lambda: torch.cat([parent[:, :4], parent[:, 4:], c, d], 1)), n * 16 * 80 * 80 * 16 * 4
    if name == "upsample2x_256x40x40":
        x = h16(n, 16, 40, 40, 16)
        return (lambda: x.repeat_interleave(2, 2).repeat_interleave(2, 3)), x.numel() * 2 * 5
    if name == "upsample_cat_256+128":
        x, y = h16(n, 16, 40, 40, 16), h16(n, 8, 80, 80, 16)
        return (lambda: torch.cat((x.repeat_interleave(2, 2).repeat_interleave(2, 3), y), 1)), \
            (x.numel() + y.numel() + n * 24 * 80 * 80 * 16) * 2
    if name == "dfl_expect_64x8400":
        x = h16(n, 64, 8400) * 3
        w = torch.arange(16, dtype=torch.float32).view(1, 1, 16, 1)
        return (lambda: (torch.softmax(x.float().view(n, 4, 16, 8400), 2) * w).sum(2).half()), \
            n * (64 + 4) * 8400 * 2
    if name == "dfl_softmax_16x4x8400":
        x = h16(n, 64, 8400) * 3
        return (lambda: torch.softmax(x.view(n, 4, 16, 8400).transpose(1, 2), 1)), x.numel() * 4
    if name == "sigmoid_80x8400":
        x = h16(n, 80, 8400)
        return (lambda: torch.sigmoid(x)), x.numel() * 4
    if name == "softmax_4x400x400":
        x = h16(n, 4, 400, 400)
        return (lambda: torch.softmax(x, -1)), x.numel() * 4
    if name == "maxpool_k5_256x20x20":
        x = h16(n, 256, 20, 20)
        return (lambda: F.max_pool2d(x.float(), 5, 1, 2).half()), x.numel() * 4
    if name == "sppf_k5x3_cat_256x20x20":
        x = h16(n, 256, 20, 20)

        def sppf():
            ys = [x]
            for _ in range(3):
                ys.append(F.max_pool2d(ys[-1].float(), 5, 1, 2).half())
            return torch.cat(ys, 1)
        return sppf, x.numel() * 2 * 5
    if name == "detect_decode_64+80x8400":
        from oracle import detect as dt  # the CPU decode sequence, timed
        b, sc = h16(n, 64, 8400) * 3, h16(n, 80, 8400)
        shapes, strides = [(80, 80), (40, 40), (20, 20)], [8.0, 16.0, 32.0]
        return (lambda: dt.detect_decode(b, sc, shapes, strides)), n * 8400 * 2 * (64 + 80 + 84)
    if name == "detect_decode_4+80x8400":
        from oracle import detect as dt  # the CPU decode sequence, timed
        b, sc = (torch.rand(n, 4, 8400, generator=g) * 20).half(), h16(n, 80, 8400)
        shapes, strides = [(80, 80), (40, 40), (20, 20)], [8.0, 16.0, 32.0]
        return (lambda: dt.detect_decode(b, sc, shapes, strides)), n * 8400 * 2 * (4 + 80 + 84)
    if name == "permute_nchw_to_nhwc_64x80x80":
        x = h16(n, 64, 80, 80)
        return (lambda: x.permute(0, 2, 3, 1).contiguous()), x.numel() * 4
    if name.startswith("attn_") or name.startswith("channel_select"):
        from oracle import bmm as ob  # the sequential-fp32 CPU contraction, timed
        heads, key, dim, tokens = ATTN
        qkv = h16(1, heads * (2 * key + dim) // 16, tokens, 16)
        if name.startswith("attn_qk"):
            return (lambda: ob.layout_bmm(qkv, qkv, True, False, False, heads, 0, key, key, key)), \
                heads * (2 * key * tokens + tokens * tokens) * 2
        if name.startswith("attn_pv"):
            p = torch.rand(heads, tokens, tokens, generator=g).half()
            return (lambda: ob.layout_bmm(qkv, p, False, True, True, heads, 2 * key, dim)), \
                heads * (2 * dim * tokens + tokens * tokens) * 2
        if name.startswith("attn_fused") or name.startswith("attn_chain"):
            from oracle import elementwise as ew  # the CPU chain, timed
            from oracle import reductions as rd
            pre = "_prescale_" in name

            def attention():
                if pre:
                    query = ew.binary_scalar_rounded(1, ob.channel_select(qkv, heads, 0, key), key ** -0.5)
                    scores = ob.layout_bmm(query, qkv, True, False, False, heads, 0, key, key, key)
                else:
                    scores = ew.binary_scalar_rounded(
                        1, ob.layout_bmm(qkv, qkv, True, False, False, heads, 0, key, key, key), key ** -0.5)
                return ob.layout_bmm(qkv, rd.softmax(scores, -1), False, True, True, heads, 2 * key, dim)
            return attention, attn_fused_bytes()
        return (lambda: ob.channel_select(qkv, heads, 2 * key, dim)), heads * dim * tokens * 2 * 2
    if name.startswith("detection_select"):
        from oracle import selection as sel  # the stable CPU selection, timed
        from tests.selection_fixtures import c5_selection_input
        x = c5_selection_input()
        return (lambda: sel.select(x, 300, False)), 8400 * 84 * 2 + 300 * 6 * 4
    return None


def time_cpu(fn, warmup=3, min_samples=20, floor_samples=5, budget_s=1.0):
    """(median seconds, sample count) of fn(): `warmup` untimed calls, then
    `min_samples` timed ones -- cut to `floor_samples` when single calls are so
    slow that the samples would run past `budget_s`."""
    for _ in range(warmup):
        fn()
    samples, t_end = [], time.perf_counter() + budget_s
    while len(samples) < min_samples and (len(samples) < floor_samples or time.perf_counter() < t_end):
        t0 = time.perf_counter_ns()
        fn()
        samples.append((time.perf_counter_ns() - t0) / 1e9)
    return statistics.median(samples), len(samples)


def cpu_baseline(budget_s=12.0):
    """The reference's CPU op sequence F.silu(torch.add(torch.mul(x, s), b)) in
    fp16 (restated by the oracle) over the same step as the GPU figure -- N=32,
    the three shapes, full and narrowed -- repeated for about `budget_s` seconds
    on the host cores.  GB/s uses the same algorithmic bytes as ``value``."""
    from oracle import elementwise as ew  # the oracle's CPU sequence, timed
    threads = torch.get_num_threads()
    n = 32
    sets, step_bytes = [], 0
    for (c, h, w) in C2_SHAPES:
        g = gen(3)
        c1 = c // 16
        x = torch.randn((n, c1, h, w, 16), generator=g).half()
        s = (torch.rand((1, c1, 1, 1, 16), generator=g) + 0.5).half()
        b = (torch.randn((1, c1, 1, 1, 16), generator=g) * 0.1).half()
        sets.append((x, s, b))
        sets.append((x[:, c1 // 2:], s[:, c1 // 2:], b[:, c1 // 2:]))
    for x, s, b in sets:
        step_bytes += (x.numel() * 2 + s.numel() * 2) * 2

    def step():
        for x, s, b in sets:
            ew.affine_silu(x, s, b)
    step()
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < budget_s:
        step()
        reps += 1
    total_s = time.perf_counter() - t0
    cpu = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(step_bytes * reps / total_s / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"the bench step on the CPU: F.silu(torch.add(torch.mul(x,s),b)) fp16, N={n}, shapes "
                      f"{C2_SHAPES} full + narrowed, {reps} steps in {total_s:.1f} s after one warm step, "
                      f"{threads} torch threads; host CPU: {cpu}"}


# ------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-ops", action="store_true", help="skip the per-op table")
    ap.add_argument("--iters", type=int, default=200, help="launches per per-op timing round")
    ap.add_argument("--profile", default=None,
                    help="replay one kernel only and print its timing (rocprofv3 summaries / counter "
                         "calibration): 'dominant', 'copy' (a plain 16-byte copy of the same size), "
                         "'copy@<C>x<H>x<W>' (a copy of one N=32 C2 tensor), 'floor' (a one-element fill: "
                         "the per-launch floor), or 'op:<row name>[@N]' for one row of the per-op table "
                         "(N=32 by default, rotated), or 'sweep' (rotated launches of plain streaming kernels "
                         "at several read:write mixes and sizes, each fitted as t = t0 + bytes / BW)")
    ap.add_argument("--ops-json", default=None, help="also write the per-op rows to this file")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the multi-GPU sharding of "
              "this path is a design note, not a measured configuration.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    from thintnpu_amd import capi
    capi.lib()
    dev = torch.device("cuda:0")
    n = 32
    if args.profile == "sweep":
        hbm_sweep(capi, dev, args.iters)
        return
    if args.profile and args.profile.startswith("op:c2f_chain_captured"):
        nn = int(args.profile.partition("@")[2] or 32)
        t = time_c2f_captured(nn, args.iters)
        print(json.dumps({"profile": f"c2f_chain_captured N={nn}", "us": round(t * 1e6, 3),
                          "GB/s": round(c2f_chain_bytes(nn) / t / 1e9, 1), "bytes": c2f_chain_bytes(nn)}))
        return
    if args.profile and args.profile.startswith("op:"):
        name, _, nn = args.profile[3:].partition("@")
        rows = [(rn, f) for (rname, _, rn, f) in op_rows(capi, dev) if rname == name]
        # default: the row's N=32 case, else its only (N=1) case
        nn = int(nn) if nn else (32 if any(rn == 32 for rn, _ in rows) else 1)
        found = [f for rn, f in rows if rn == nn]
        if not found:
            print(f"no op row {name!r} at N={nn}", file=sys.stderr)
            sys.exit(2)
        launch, sets, algo = found[0](not name.startswith("detection_select"))
        t = time_launches(launch, sets, args.iters)
        print(json.dumps({"profile": f"{name} N={nn}", "us": round(t * 1e6, 3), "GB/s": round(algo / t / 1e9, 1),
                          "bytes": algo}))
        return
    if args.profile == "floor":
        # the per-launch floor: a one-element thin_fill (one block) replayed
        # back to back from a HIP graph like every row
        sets = [torch.empty(1, dtype=torch.float16, device=dev) for _ in range(2)]
        t = time_launches(lambda st: capi.fill(st, 1.0), sets, args.iters)
        print(json.dumps({"profile": "thin_fill of one fp16 element (one block)", "us": round(t * 1e6, 3)}))
        return
    if args.profile and args.profile.startswith("copy@"):
        # a plain copy of the bytes of one C2 launch: [32,C/16,H,W,16] fp16
        c, h, w = (int(v) for v in args.profile[5:].split("x"))
        per = n * (c // 16) * h * w * 16 * 2
        sets = rotated(lambda i: (blocked_normal(n, c, h, w, 800 + i, dev),
                                  torch.empty((n, c // 16, h, w, 16), dtype=torch.float16, device=dev)), 2 * per, True)
        t = time_launches(lambda st: capi.copy(st[0], st[1]), sets, args.iters)
        print(json.dumps({"profile": f"copy of [{n},{c // 16},{h},{w},16] fp16", "us": round(t * 1e6, 3),
                          "GB/s": round(2 * per / t / 1e9, 1), "bytes": 2 * per}))
        return
    if args.profile:
        if args.profile not in ("dominant", "copy"):
            print(f"unknown --profile {args.profile!r}", file=sys.stderr)
            sys.exit(2)
        launch, sets, algo = op_affine_silu(capi, dev, n, *C2_SHAPES[0], False, rotate=True)
        what = "affine_silu N=32 C,H,W=(128,80,80)"
        if args.profile == "copy":
            sets = [(st[0], st[3]) for st in sets]
            launch = lambda st: capi.copy(st[0], st[1])  # noqa: E731
            what = "copy of the same [32,8,80,80,16] fp16 tensor (104857600 B read + written)"
            algo = 2 * sets[0][0].numel() * 2
        t = time_launches(launch, sets, args.iters)
        print(json.dumps({"profile": what, "us": round(t * 1e6, 3),
                          "GB/s": round(algo / t / 1e9, 1), "launches": args.iters * 6 + 3}))
        return

    # ---- the step: six affine_silu launches at N=32 with rotated buffer sets
    work = []
    for (c, h, w) in C2_SHAPES:
        for narrowed in (False, True):
            work.append(op_affine_silu(capi, dev, n, c, h, w, narrowed, rotate=False))
    step_bytes = sum(a for _, _, a in work)
    per_set = sum(sum(t.numel() * t.element_size() for t in sets[0]) for _, sets, _ in work)
    nrot = rotation_count(per_set)
    rot_sets = [[op_affine_silu(capi, dev, n, c, h, w, nr, rotate=False)[1][0]
                 for (c, h, w) in C2_SHAPES for nr in (False, True)] for _ in range(nrot)]

    def step_launches(sets):
        for (launch, _, _), st in zip(work, sets):
            launch(st)

    for sets in rot_sets:  # eager warm pass
        step_launches(sets)
    torch.cuda.synchronize()
    # Step i runs on rotated set i % nrot.  Runs of GRAPH_STEPS consecutive
    # steps replay one HIP graph holding all of their launches (a graph launch
    # between every step costs ~4 us of idle device time: 60.5 against 56.3 us
    # per step); leftover steps replay one-step graphs.
    graphs1 = [capture(lambda r=r: step_launches(rot_sets[r])) for r in range(nrot)]
    graphs_g = [capture(lambda r=r: [step_launches(rot_sets[(r + j) % nrot]) for j in range(GRAPH_STEPS)])
                for r in range(nrot)]

    def run_steps(first, count):
        i, end = first, first + count
        while i < end:
            if end - i >= GRAPH_STEPS:
                graphs_g[i % nrot].replay()
                i += GRAPH_STEPS
            else:
                graphs1[i % nrot].replay()
                i += 1

    log(f"step: {len(work)} launches, {step_bytes / 1e6:.1f} MB algorithmic, {nrot} rotated sets, "
        f"{GRAPH_STEPS} steps per graph replay")
    run_steps(0, args.warmup)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    run_steps(args.warmup, args.steps)
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_s = start.elapsed_time(stop) / 1e3 / args.steps
    value = step_bytes / step_s / 1e9
    log(f"step {step_s * 1e6:.1f} us  {value:.1f} GB/s  (wall {wall:.3f} s)")

    # ---- roofline of the dominant kernel: affine_silu on the largest shape, N=32
    launch, sets, algo = op_affine_silu(capi, dev, n, *C2_SHAPES[0], False, rotate=True)
    dom_s = time_launches(launch, sets, args.iters)
    achieved = algo / dom_s / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": dominant_traffic(),
                "kernel": "affine_silu_flat_kernel<2, true, true> (thin_affine_silu)",
                "launch": f"N=32 C,H,W={C2_SHAPES[0]}: {algo} algorithmic bytes, avg {dom_s * 1e6:.2f} us",
                "traffic_note": "HBM bytes per launch = sum of L2-to-HBM read and write requests x their "
                                "sizes (rocprofv3 --pmc TCC_EA0_RDREQ_32B/_64B/_128B, TCC_EA0_WRREQ/_64B; "
                                "profiles/affine_silu_flat_n32_128x80x80_pmc.md)"}
    del sets

    ops = []
    if not args.no_ops:
        for name, cfg, nn, factory in op_rows(capi, dev):
            modes = (False,) if name.startswith("detection_select") else ((False, True) if nn == 1 else (True,))
            cpu_row = None
            if not args.no_cpu:
                made = cpu_op(name, nn)
                if made is not None:
                    fn, cpu_bytes = made
                    threads = torch.get_num_threads()
                    ct, ns = time_cpu(fn)
                    torch.set_num_threads(1)  # the reference tests' thread count
                    try:
                        ct1, ns1 = time_cpu(fn)
                    finally:
                        torch.set_num_threads(threads)
                    cpu_row = {"cpu_us": round(ct * 1e6, 1), "cpu_GB/s": round(cpu_bytes / ct / 1e9, 2),
                               "cpu_threads": threads, "cpu_samples": ns,
                               "cpu1_us": round(ct1 * 1e6, 1), "cpu1_GB/s": round(cpu_bytes / ct1 / 1e9, 2),
                               "cpu1_samples": ns1}
                    del fn
            for rotate in modes:
                launch, sets, algo = factory(rotate)
                t = time_launches(launch, sets, args.iters)
                gbs = algo / t / 1e9
                row = {"op": name, "cfg": cfg, "N": nn, "us": round(t * 1e6, 3),
                       "GB/s": round(gbs, 1), "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
                       "bytes": algo, "cache": "rotated" if rotate else "resident"}
                if cpu_row:
                    row.update(cpu_row)
                ops.append(row)
                log(f"{cfg} {name:32s} N={nn:2d} {'rot' if rotate else 'res'} "
                    f"{t * 1e6:9.2f} us {gbs:8.1f} GB/s" +
                    (f"   cpu {cpu_row['cpu_us']:10.1f} us  1 thread {cpu_row['cpu1_us']:10.1f} us"
                     if cpu_row else ""))
                del sets
                torch.cuda.empty_cache()

        # the drop-in path as callers use it: a CapturedForward-replayed C2f
        # tail on the npu device (wall clock per replay)
        for nn in (1, 32):
            cpu_row = None
            if not args.no_cpu:
                fn, cpu_bytes = cpu_op("c2f_chain_captured", nn)
                ct, ns = time_cpu(fn)
                cpu_row = {"cpu_us": round(ct * 1e6, 1), "cpu_GB/s": round(cpu_bytes / ct / 1e9, 2),
                           "cpu_threads": torch.get_num_threads(), "cpu_samples": ns}
                del fn
            for rotate in ((False, True) if nn == 1 else (True,)):
                t = time_c2f_captured(nn, args.iters, rotate=rotate)
                algo = c2f_chain_bytes(nn)
                gbs = algo / t / 1e9
                row = {"op": "c2f_chain_captured", "cfg": "C2f", "N": nn, "us": round(t * 1e6, 3),
                       "GB/s": round(gbs, 1), "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 1), "bytes": algo,
                       "cache": "rotated" if rotate else "resident",
                       "note": "CapturedForward replay on npu (split, silu_, add, cat), wall clock per replay"}
                if cpu_row:
                    row.update(cpu_row)
                ops.append(row)
                log(f"C2f {'c2f_chain_captured':32s} N={nn:2d} {'rot' if rotate else 'res'} "
                    f"{t * 1e6:9.2f} us {gbs:8.1f} GB/s")
                torch.cuda.empty_cache()

    cpu = None if args.no_cpu else cpu_baseline()
    # The per-op table goes to stderr, one JSON object per row, and to
    # --ops-json when given; stdout's last line is the compact headline.
    for row in ops:
        log(json.dumps(row))
    if args.ops_json:
        Path(args.ops_json).parent.mkdir(parents=True, exist_ok=True)
        Path(args.ops_json).write_text(json.dumps(ops, indent=1) + "\n")
    line = headline(value=value, step_s=step_s, steps=args.steps, warmup=args.warmup, batch=n,
                    launches=len(work), step_bytes=step_bytes, nrot=nrot, roofline=roofline, cpu=cpu,
                    op_rows=len(ops))
    print(json.dumps(line), flush=True)


HEADLINE_MAX_BYTES = 4096  # the driver reads the tail of stdout; the last line must fit in it whole


def headline(*, value, step_s, steps, warmup, batch, launches, step_bytes, nrot, roofline, cpu, op_rows):
    """The bench's last stdout line: the step's throughput, its roofline and
    CPU baseline, in a few KB (the per-op rows are printed on stderr)."""
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "affine+SiLU y=SiLU(x*s+b), per-channel [1,C,1,1] broadcast, NC1HWC0 fp16, "
                               "N=32, (C,H,W) in {(128,80,80),(256,40,40),(512,20,20)}, full + C2f "
                               "narrowed view x[:,C/2:]",
                   "batch": batch, "shapes": C2_SHAPES, "launches_per_step": launches,
                   "algorithmic_bytes_per_step": step_bytes, "rotated_sets": nrot,
                   "steps_per_graph": GRAPH_STEPS},
        "pct_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ops_rows": op_rows,
        "ops_where": "stderr, one JSON object per row (and --ops-json)",
    }
    # never fail at the end of a run: shorten the free-text fields until it fits
    for holder, key in ((roofline, "traffic_note"), (cpu, "sample"), (roofline, "launch")):
        excess = len(json.dumps(line)) - HEADLINE_MAX_BYTES
        if excess <= 0:
            break
        if isinstance(holder, dict) and isinstance(holder.get(key), str):
            text = holder[key]
            holder[key] = text[:max(0, len(text) - excess - 3)] + "..."
    return line


if __name__ == "__main__":
    main()

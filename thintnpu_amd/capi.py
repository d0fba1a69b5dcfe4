"""ctypes binding of the C ABI in include/thin_hip.h.

Device memory and streams come from PyTorch's HIP device (``torch.cuda``):
a tensor's ``data_ptr()`` (storage offset included), sizes and strides fill a
``thin_desc``; the stream is ``torch.cuda.current_stream()``.  The binding
loads ``libthin_hip.so`` only after ``import torch`` so that the library
shares the HIP runtime torch already loaded (both carry the soname
libamdhip64.so.7).  A missing library raises: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libthin_hip.so"
MAX_DIMS = 8
MAX_CAT_INPUTS = 64

F16, F32, I64, I32, I16, U8, F64, BF16 = range(8)
SELECT_SCRATCH_BYTES = 8 << 20  # THIN_SELECT_SCRATCH_BYTES of include/thin_hip.h
SUB, MUL, DIV, ADD = 0, 1, 2, 3
SIGMOID, SILU = 0, 1

_DTYPES = {
    torch.float16: F16, torch.float32: F32, torch.int64: I64, torch.int32: I32,
    torch.int16: I16, torch.uint8: U8, torch.float64: F64, torch.bfloat16: BF16,
    torch.int8: U8, torch.bool: U8,  # byte-sized: moved and filled as raw bytes
}
STATUS = {0: "THIN_OK", 1: "THIN_ERR_INVALID", 2: "THIN_ERR_UNSUPPORTED", 3: "THIN_ERR_HIP",
          4: "THIN_ERR_WORKSPACE"}


class ThinDesc(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("sizes", ctypes.c_int64 * MAX_DIMS),
        ("strides", ctypes.c_int64 * MAX_DIMS),
    ]


class ThinSelectTrace(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("class_max", "stage1", "gathered", "top_values", "stage2", "anchors", "labels")]


class ThinBmmLayout(ctypes.Structure):
    _fields_ = [("transpose_a", ctypes.c_int32), ("transpose_b", ctypes.c_int32),
                ("blocked_output", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("groups", ctypes.c_int64), ("a_offset", ctypes.c_int64), ("a_channels", ctypes.c_int64),
                ("b_offset", ctypes.c_int64), ("b_channels", ctypes.c_int64)]


class ThinError(RuntimeError):
    """A C-ABI call returned a non-zero thin_status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn}: {STATUS.get(status, status)}: {message}")
        self.status = status


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run python -m thintnpu_amd.build")
        L = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
        P = ctypes.POINTER(ThinDesc)
        vp, i32, i64, f32, f64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        sigs = {
            "thin_binary": [i32, P, P, P, f32, vp],
            "thin_binary_scalar": [i32, P, f64, i32, P, f32, vp],
            "thin_unary": [i32, P, P, vp],
            "thin_silu_add": [P, P, P, vp],
            "thin_affine_silu": [P, P, P, P, vp],
            "thin_copy": [P, P, vp],
            "thin_cat": [P, i32, i32, P, vp],
            "thin_upsample2x_nc1hwc0": [P, P, vp],
            "thin_upsample2x_nchw": [P, P, vp],
            "thin_upsample_cat_nc1hwc0": [P, ctypes.POINTER(i32), i32, P, vp],
            "thin_pack_nc1hwc0": [P, P, vp],
            "thin_unpack_nc1hwc0": [P, P, vp],
            "thin_softmax": [P, i32, P, vp],
            "thin_dfl_expect": [P, P, vp],
            "thin_maxpool_nc1hwc0": [P, i32, P, vp],
            "thin_sppf_nc1hwc0": [P, i32, i32, P, vp],
            "thin_maxpool2d_nchw": [P, i32, P, vp],
            "thin_fill": [P, f64, i64, vp],
            "thin_detect_decode": [P, P, ctypes.POINTER(i32), ctypes.POINTER(f64), i32, i32, P, vp],
            "thin_detection_select": [P, i64, i32, vp, vp, ctypes.c_size_t,
                                      ctypes.POINTER(ThinSelectTrace), vp],
            "thin_detection_select_noalloc": [P, i64, i32, vp, ctypes.POINTER(ThinSelectTrace), vp],
            "thin_layout_bmm_shape": [P, P, ctypes.POINTER(ThinBmmLayout), ctypes.POINTER(i32),
                                      ctypes.POINTER(i64)],
            "thin_layout_bmm": [P, P, ctypes.POINTER(ThinBmmLayout), P, vp],
            "thin_channel_select_shape": [P, i64, i64, i64, ctypes.POINTER(i64)],
            "thin_channel_select": [P, i64, i64, i64, P, vp],
            "thin_attention": [P, i64, i64, i64, ctypes.c_float, i32, P, vp],
        }
        for name, argtypes in sigs.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        L.thin_last_error.restype = ctypes.c_char_p
        L.thin_version.restype = ctypes.c_char_p
        if hasattr(L, "thin_detection_select_workspace"):
            L.thin_detection_select_workspace.argtypes = [i64, i64, i64, i64, i32]
            L.thin_detection_select_workspace.restype = ctypes.c_size_t
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    """Names declared in include/thin_hip.h that the loaded library exports."""
    L = lib()
    return [n for n in declared_symbols() if hasattr(L, n)]


def declared_symbols() -> list[str]:
    import re
    header = (Path(__file__).resolve().parent.parent / "include" / "thin_hip.h").read_text()
    return sorted(set(re.findall(r"\b(thin_[a-z0-9_]+)\s*\(", header)))


def desc(t: torch.Tensor) -> ThinDesc:
    if t.dim() > MAX_DIMS:
        raise ValueError(f"rank {t.dim()} exceeds {MAX_DIMS}")
    d = ThinDesc()
    d.data = t.data_ptr() if t.numel() else 0
    d.dtype = _DTYPES[t.dtype]
    d.rank = t.dim()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        d.sizes[i] = s
        d.strides[i] = st
    return d


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


def _check(fn: str, status: int) -> None:
    if status != 0:
        raise ThinError(fn, status, lib().thin_last_error().decode())


def _call(name: str, *args) -> None:
    _check(name, getattr(lib(), name)(*args))


def _ref(d: ThinDesc):
    return ctypes.byref(d)


# ----------------------------------------------------------------- wrappers
# Each wrapper allocates its output with torch on the input's device (tests and
# the bench own the memory); the library itself never allocates.

def binary(op: int, x: torch.Tensor, y: torch.Tensor, alpha: float = 1.0, out=None, stream=None):
    shape = torch.broadcast_shapes(x.shape, y.shape)
    xe, ye = x.expand(shape), y.expand(shape)
    out = torch.empty(shape, dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_binary", op, _ref(desc(xe)), _ref(desc(ye)), _ref(desc(out)), alpha, _stream(stream))
    return out


def binary_scalar(op: int, x: torch.Tensor, scalar: float, scalar_first: bool = False,
                  alpha: float = 1.0, out=None, stream=None):
    out = torch.empty_like(x, memory_format=torch.contiguous_format) if out is None else out
    _call("thin_binary_scalar", op, _ref(desc(x)), float(scalar), int(scalar_first),
          _ref(desc(out)), alpha, _stream(stream))
    return out


def unary(op: int, x: torch.Tensor, out=None, stream=None):
    out = torch.empty_like(x, memory_format=torch.contiguous_format) if out is None else out
    _call("thin_unary", op, _ref(desc(x)), _ref(desc(out)), _stream(stream))
    return out


def silu_add(x, y, out=None, stream=None):
    shape = torch.broadcast_shapes(x.shape, y.shape)
    out = torch.empty(shape, dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_silu_add", _ref(desc(x.expand(shape))), _ref(desc(y.expand(shape))),
          _ref(desc(out)), _stream(stream))
    return out


def affine_silu(x, s, b, out=None, stream=None):
    shape = x.shape
    out = torch.empty(shape, dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_affine_silu", _ref(desc(x)), _ref(desc(s.expand(shape))), _ref(desc(b.expand(shape))),
          _ref(desc(out)), _stream(stream))
    return out


def copy(src, dst, stream=None):
    _call("thin_copy", _ref(desc(src)), _ref(desc(dst)), _stream(stream))
    return dst


def cat(tensors, dim: int, out=None, stream=None):
    ref = tensors[0]
    dim = dim % ref.dim()
    shape = list(ref.shape)
    shape[dim] = sum(t.shape[dim] for t in tensors)
    out = torch.empty(shape, dtype=ref.dtype, device=ref.device) if out is None else out
    arr = (ThinDesc * len(tensors))(*[desc(t) for t in tensors])
    _call("thin_cat", arr, len(tensors), dim, _ref(desc(out)), _stream(stream))
    return out


def upsample2x_nc1hwc0(x, out=None, stream=None):
    n, c1, h, w, c0 = x.shape
    out = torch.empty((n, c1, 2 * h, 2 * w, c0), dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_upsample2x_nc1hwc0", _ref(desc(x)), _ref(desc(out)), _stream(stream))
    return out


def upsample2x_nchw(x, out=None, stream=None):
    n, c, h, w = x.shape
    out = torch.empty((n, c, 2 * h, 2 * w), dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_upsample2x_nchw", _ref(desc(x)), _ref(desc(out)), _stream(stream))
    return out


def upsample_cat_nc1hwc0(tensors, upsample, out=None, stream=None):
    ref_i = next(i for i, u in enumerate(upsample) if not u) if not all(upsample) else 0
    ref = tensors[ref_i]
    scale = 2 if upsample[ref_i] else 1
    n, _, h, w, c0 = ref.shape
    c1 = sum(t.shape[1] for t in tensors)
    out = torch.empty((n, c1, h * scale, w * scale, c0), dtype=ref.dtype, device=ref.device) \
        if out is None else out
    arr = (ThinDesc * len(tensors))(*[desc(t) for t in tensors])
    ups = (ctypes.c_int32 * len(tensors))(*[int(bool(u)) for u in upsample])
    _call("thin_upsample_cat_nc1hwc0", arr, ups, len(tensors), _ref(desc(out)), _stream(stream))
    return out


def pack_nc1hwc0(x, out=None, stream=None):
    n, c, h, w = x.shape
    out = torch.empty((n, (c + 15) // 16, h, w, 16), dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_pack_nc1hwc0", _ref(desc(x)), _ref(desc(out)), _stream(stream))
    return out


def unpack_nc1hwc0(x, channels: int | None = None, out=None, stream=None):
    n, c1, h, w, c0 = x.shape
    c = c1 * c0 if channels is None else channels
    out = torch.empty((n, c, h, w), dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_unpack_nc1hwc0", _ref(desc(x)), _ref(desc(out)), _stream(stream))
    return out


def maxpool_nc1hwc0(x, kernel: int, out=None, stream=None):
    """Stride-1 k x k max pool with padding k//2 on NC1HWC0 fp16."""
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_maxpool_nc1hwc0", _ref(desc(x)), kernel, _ref(desc(out)), _stream(stream))
    return out


def sppf_nc1hwc0(x, kernel: int = 5, repeats: int = 3, out=None, stream=None):
    """cat([x, p(x), p(p(x)), ...], 1) with p the stride-1 k x k max pool, on
    NC1HWC0 fp16 (the SPPF block's pooling and concat)."""
    n, c1, h, w, c0 = x.shape
    out = torch.empty((n, (repeats + 1) * c1, h, w, c0), dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_sppf_nc1hwc0", _ref(desc(x)), kernel, repeats, _ref(desc(out)), _stream(stream))
    return out


def maxpool2d_nchw(x, kernel: int, out=None, stream=None):
    """Stride-1 k x k max pool with padding k//2 on NCHW fp16/fp32."""
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device) if out is None else out
    _call("thin_maxpool2d_nchw", _ref(desc(x)), kernel, _ref(desc(out)), _stream(stream))
    return out


def fill(t, value, stream=None):
    """t[...] = value in place (any strides)."""
    ival = int(value) if not t.is_floating_point() else 0
    _call("thin_fill", _ref(desc(t)), float(value), ival, _stream(stream))
    return t


def softmax(x, dim: int, half_to_float: bool = False, out=None, stream=None):
    dtype = torch.float32 if half_to_float else x.dtype
    out = torch.empty(x.shape, dtype=dtype, device=x.device) if out is None else out
    _call("thin_softmax", _ref(desc(x)), dim % max(1, x.dim()), _ref(desc(out)), _stream(stream))
    return out


def dfl_expect(x, out_dtype=None, out=None, stream=None):
    n, c, a = x.shape
    out = torch.empty((n, c // 16, a), dtype=out_dtype or x.dtype, device=x.device) if out is None else out
    _call("thin_dfl_expect", _ref(desc(x)), _ref(desc(out)), _stream(stream))
    return out


def detect_decode(boxes, scores, shapes, strides, xywh: bool = False, out=None, stream=None):
    """Anchor-free head decode: [B,64,A] box logits (or [B,4,A] distances of a
    reg_max = 1 head) + [B,nc,A] class logits -> [B,4+nc,A] fp16 (boxes by DFL
    (or as given) + grid + stride, scores by sigmoid).
    shapes: per-level (h, w); strides: per-level stride."""
    b, _, a = boxes.shape
    nc = scores.shape[1]
    out = torch.empty((b, 4 + nc, a), dtype=torch.float16, device=boxes.device) if out is None else out
    levels = len(shapes)
    hw = (ctypes.c_int32 * (2 * levels))(*[int(v) for hw_ in shapes for v in hw_])
    st = (ctypes.c_double * levels)(*[float(v) for v in strides])
    _call("thin_detect_decode", _ref(desc(boxes)), _ref(desc(scores)), hw, st, levels, int(xywh),
          _ref(desc(out)), _stream(stream))
    return out


def detection_select_workspace(b: int, a: int, nc: int, max_det: int, agnostic: bool) -> int:
    return int(lib().thin_detection_select_workspace(b, a, nc, max_det, int(agnostic)))


def detection_select(decoded, max_det: int, agnostic: bool = False, trace: bool = False,
                     stream=None, out=None, workspace=None, noalloc: bool = False):
    """thin_detection_select with a workspace (given, or allocated here), or,
    with noalloc=True, thin_detection_select_noalloc on the library's static
    scratch (no workspace argument).  trace: True for every trace stage, or
    a collection of stage names for those only (the others stay null)."""
    b, a, ch = decoded.shape
    nc = ch - 4
    k = min(max_det, a)
    dev = decoded.device
    out = torch.empty((b, k, 6), dtype=torch.float32, device=dev) if out is None else out
    ws = None
    if not noalloc:
        ws_bytes = detection_select_workspace(b, a, nc, max_det, agnostic)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if workspace is None else workspace
    tr = None
    tensors = None
    if trace:
        tensors = dict(
            class_max=torch.empty((b, a), dtype=torch.float16, device=dev),
            stage1=torch.empty((b, k), dtype=torch.int64, device=dev),
            gathered=torch.empty((b, 0 if agnostic else k, nc), dtype=torch.float16, device=dev),
            top_values=torch.empty((b, k), dtype=torch.float16, device=dev),
            stage2=torch.empty((b, 0 if agnostic else k), dtype=torch.int64, device=dev),
            anchors=torch.empty((b, k), dtype=torch.int64, device=dev),
            labels=torch.empty((b, k), dtype=torch.int64, device=dev),
        )
        if trace is not True:
            tensors = {n: t for n, t in tensors.items() if n in set(trace)}
        tr = ThinSelectTrace(**{n: (t.data_ptr() if t.numel() else None) for n, t in tensors.items()})
    trace_arg = ctypes.byref(tr) if tr is not None else None
    out_ptr = out.data_ptr() if out.numel() else None
    if noalloc:
        _call("thin_detection_select_noalloc", _ref(desc(decoded)), max_det, int(agnostic), out_ptr, trace_arg,
              _stream(stream))
    else:
        _call("thin_detection_select", _ref(desc(decoded)), max_det, int(agnostic), out_ptr, ws.data_ptr(),
              ws.numel(), trace_arg, _stream(stream))
    if trace:
        return out, tensors
    return out


def layout_bmm(a, b, transpose_a: bool = False, transpose_b: bool = False, blocked_output: bool = False,
               groups: int = 0, a_offset: int = 0, a_channels: int = -1, b_offset: int = 0, b_channels: int = -1,
               out=None, stream=None):
    """a @ b over the logical fp16 matrices of rank-3 or channel-blocked
    rank-4 operands (head groups, channel ranges, transposes), summed in fp32
    in reduction order.  Unblocked results are the [.., :n] view of a buffer
    whose rows are n rounded up to 16 columns, as the reference returns them."""
    L = ThinBmmLayout(int(transpose_a), int(transpose_b), int(blocked_output), 0, groups, a_offset, a_channels,
                      b_offset, b_channels)
    rank = ctypes.c_int32()
    sizes = (ctypes.c_int64 * 4)()
    _call("thin_layout_bmm_shape", _ref(desc(a)), _ref(desc(b)), ctypes.byref(L), ctypes.byref(rank), sizes)
    shape = tuple(sizes[:rank.value])
    if out is None:
        if blocked_output:
            out = torch.empty(shape, dtype=torch.float16, device=a.device)
        else:
            n = shape[2]
            out = torch.empty((shape[0], shape[1], (n + 15) // 16 * 16), dtype=torch.float16,
                              device=a.device)[:, :, :n]
    _call("thin_layout_bmm", _ref(desc(a)), _ref(desc(b)), ctypes.byref(L), _ref(desc(out)), _stream(stream))
    return out


def bmm(a, b, out=None, stream=None):
    """Rank-3 a @ b (fp16, any strides), fp32 sums in reduction order."""
    return layout_bmm(a, b, out=out, stream=stream)


def channel_select(x, groups: int, begin: int, count: int, out=None, stream=None):
    """Channels [begin, begin+count) of each of `groups` equal channel groups of
    an N=1 blocked [1, C1, T, 16] fp16 tensor, packed back to back."""
    sizes = (ctypes.c_int64 * 4)()
    _call("thin_channel_select_shape", _ref(desc(x)), groups, begin, count, sizes)
    out = torch.empty(tuple(sizes), dtype=torch.float16, device=x.device) if out is None else out
    _call("thin_channel_select", _ref(desc(x)), groups, begin, count, _ref(desc(out)), _stream(stream))
    return out


def attention(qkv, heads: int, key_dim: int, head_dim: int, scale: float, prescale: bool = True, out=None,
              stream=None):
    """Fused blocked attention of a head-grouped [1, C1, T, 16] QKV tensor:
    mixed values [1, heads * head_dim / 16, T, 16], the bits of
    channel_select -> mul -> layout_bmm -> softmax -> layout_bmm (prescale) or
    layout_bmm -> mul -> softmax -> layout_bmm.  `scale` multiplies in fp32;
    pass the fp16-rounded value for the reference's 0-d operand rule.  Shapes
    outside the fused kernel's range raise ThinError (THIN_ERR_UNSUPPORTED)."""
    tokens = qkv.shape[2]
    if out is None:
        out = torch.empty((1, heads * head_dim // 16, tokens, 16), dtype=torch.float16, device=qkv.device)
    _call("thin_attention", _ref(desc(qkv)), heads, key_dim, head_dim, float(scale), int(bool(prescale)),
          _ref(desc(out)), _stream(stream))
    return out

"""CPU checks of the boundary: the C header is plain C, libthin_hip.so loads
and exports every entry point the header declares, argument validation
rejects bad descriptors before any device work, and the PrivateUse1 glue
libraries register their kernels.  Nothing here launches a kernel."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

from thintnpu_amd import capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "thin_hip.h"


def test_header_is_plain_c(tmp_path):
    """The boundary compiles as C11 (no C++ or torch types leak into it)."""
    src = tmp_path / "abi.c"
    src.write_text('#include "thin_hip.h"\n'
                   "int main(void) { thin_desc d; thin_select_trace t; (void)d; (void)t;\n"
                   "  return (int)sizeof(thin_desc) != 8 + 4 + 4 + 8 * 8 * 2; }\n")
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{ROOT / 'include'}",
                    "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", str(src), "-o", str(tmp_path / "abi")],
                   check=True)
    assert subprocess.run([str(tmp_path / "abi")]).returncode == 0


def test_library_exports_every_declared_symbol():
    declared = capi.declared_symbols()
    assert len(declared) >= 17
    lib = capi.lib()
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.thin_version().decode().startswith("thin-hip")


def test_every_declaration_cites_the_reference():
    """Each entry point's comment names the reference interface it replaces."""
    text = HEADER.read_text()
    for name in capi.declared_symbols():
        if name in ("thin_last_error", "thin_version"):
            continue
        start = text.index(name + "(")
        comment = text[text.rfind("/*", 0, start):start]
        if "No counterpart in the reference" in comment:
            assert "cannot allocate" in " ".join(comment.replace("*", " ").split()), name  # the allocation-free variant names its callers
            continue
        assert re.search(r"\w+\.(cpp|py|h):\d+", comment), name


def desc_of(shape, dtype=capi.F16, data=0x1000, strides=None):
    d = capi.ThinDesc()
    d.data = data
    d.dtype = dtype
    d.rank = len(shape)
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, strides)):
        d.sizes[i], d.strides[i] = s, st
    return d


def status_of(name, *args):
    lib = capi.lib()
    code = getattr(lib, name)(*args)
    return code, lib.thin_last_error().decode()


P = ctypes.byref


@pytest.mark.parametrize("case", ["null", "dtype", "shape", "rank", "op"])
def test_binary_validation(case):
    x, y, out = desc_of((2, 3)), desc_of((2, 3)), desc_of((2, 3))
    if case == "null":
        code, msg = status_of("thin_binary", capi.ADD, None, P(y), P(out), 1.0, None)
    else:
        if case == "dtype":
            x = desc_of((2, 3), capi.I64)
        elif case == "shape":
            y = desc_of((3, 3))
        elif case == "rank":
            x.rank = 9
        op = 17 if case == "op" else capi.ADD
        code, msg = status_of("thin_binary", op, P(x), P(y), P(out), 1.0, None)
    assert code in (1, 2), (case, code, msg)
    assert msg


def test_movement_validation():
    a, b = desc_of((1, 2, 4, 4, 16)), desc_of((1, 3, 4, 4, 16))
    arr = (capi.ThinDesc * 2)(a, b)
    bad_out = desc_of((1, 6, 4, 4, 16))
    code, msg = status_of("thin_cat", arr, 2, 1, P(bad_out), None)
    assert code == 1 and "cat" in msg
    code, msg = status_of("thin_cat", arr, 65, 1, P(bad_out), None)
    assert code == 1
    code, msg = status_of("thin_upsample2x_nc1hwc0", P(a), P(desc_of((1, 2, 8, 9, 16))), None)
    assert code == 1
    code, msg = status_of("thin_pack_nc1hwc0", P(desc_of((1, 17, 4, 4))), P(desc_of((1, 1, 4, 4, 16))), None)
    assert code == 1
    code, msg = status_of("thin_softmax", P(desc_of((2, 5))), 2, P(desc_of((2, 5))), None)
    assert code == 1
    code, msg = status_of("thin_dfl_expect", P(desc_of((1, 63, 10))), P(desc_of((1, 4, 10))), None)
    assert code == 1


def test_selection_workspace_and_validation():
    lib = capi.lib()
    small = lib.thin_detection_select_workspace(1, 8400, 80, 300, 0)
    big = lib.thin_detection_select_workspace(2, 8400, 80, 300, 0)
    assert 0 < small < big
    assert lib.thin_detection_select_workspace(1, 8400, 80, 9000, 0) > small
    out = desc_of((1, 300, 6), capi.F32)
    code, msg = status_of("thin_detection_select", P(desc_of((1, 8400, 84))), 300, 0, P(out), None,
                          ctypes.c_size_t(0), None, None)
    assert code in (1, 4) and msg


def test_glue_registers_privateuse1():
    import thin_backend
    thin_backend.load_flow_libraries()
    assert torch._C._get_privateuse1_backend_name() == "npu"
    has = torch._C._dispatch_has_kernel_for_dispatch_key
    for op in ("aten::add.Tensor", "aten::sub.Tensor", "aten::mul.Tensor", "aten::div.Tensor",
               "aten::sigmoid", "aten::silu", "aten::silu_", "aten::cat", "aten::_softmax",
               "aten::upsample_nearest2d", "aten::copy_", "aten::empty.memory_format", "aten::empty_strided",
               "aten::as_strided", "aten::view", "aten::split.Tensor", "aten::convolution",
               "thin_backend::add", "thin_backend::sigmoid", "thin_backend::upsample_nearest2d",
               "thin_fused::silu_add", "thin_fused::affine_silu", "thin_fused::upsample_cat",
               "thin_fused::dfl_expect", "thin_fused::detect_decode", "thin_fused::sppf", "thin_native_flow::upsample",
               "thin_native_flow::pack_input", "thin_native_flow::maxpool", "thin_backend::maxpool2d",
               "aten::max_pool2d_with_indices", "aten::fill_.Scalar", "aten::zero_",
               "thin_native_flow::detection_select", "thin_native_flow::detection_select_trace",
               "thin_blocked::pack", "thin_blocked::unpack", "aten::split_with_sizes", "aten::arange.start_out",
               "aten::arange.out", "aten::_local_scalar_dense", "aten::bmm", "thin_backend::nms",
               "thin_backend::conv2d", "thin_native_flow::conv", "thin_native_flow::stem",
               "thin_native_flow::bmm", "thin_native_flow::layout_bmm", "thin_native_flow::channel_select",
               "thin_native_flow::depthwise", "thin_blocked::conv"):
        assert has(op, "PrivateUse1"), op
    assert hasattr(torch.classes.thin_backend, "RuntimeGraph")
    # plan takes no tensors: a catch-all kernel, as conv_flow.cpp:631 defines it
    assert has("thin_native_flow::plan", "CompositeImplicitAutograd")
    for op in ("thin_backend::add", "thin_backend::sigmoid", "thin_backend::upsample_nearest2d",
               "thin_backend::maxpool2d"):
        assert has(op, "Meta"), op


def test_fused_meta_shapes():
    import thin_backend  # noqa: F401
    x = torch.empty(2, 4, 8, 8, 16, dtype=torch.float16, device="meta")
    s = torch.empty(1, 4, 1, 1, 16, dtype=torch.float16, device="meta")
    assert torch.ops.thin_fused.affine_silu(x, s, s).shape == x.shape
    assert torch.ops.thin_fused.silu_add(x, x).shape == x.shape
    up = torch.empty(2, 2, 4, 4, 16, dtype=torch.float16, device="meta")
    assert torch.ops.thin_fused.upsample_cat([up, x], [1, 0]).shape == (2, 6, 8, 8, 16)
    d = torch.empty(2, 64, 100, dtype=torch.float16, device="meta")
    assert torch.ops.thin_fused.dfl_expect(d).shape == (2, 4, 100)
    assert torch.ops.thin_fused.dfl_expect(d, True).dtype == torch.float32
    b = torch.empty(2, 64, 21, dtype=torch.float16, device="meta")
    sc = torch.empty(2, 3, 21, dtype=torch.float16, device="meta")
    assert torch.ops.thin_fused.detect_decode(b, sc, [3, 5, 2, 3], [8.0, 16.0]).shape == (2, 7, 21)
    assert torch.ops.thin_fused.sppf(x).shape == (2, 16, 8, 8, 16)
    assert torch.ops.thin_fused.sppf(x, 3, 1).shape == (2, 8, 8, 8, 16)


def test_no_cpu_fallback_without_library(monkeypatch, tmp_path):
    """The binding refuses to run when the HIP library is absent."""
    monkeypatch.setattr(capi, "LIB_PATH", tmp_path / "missing.so")
    monkeypatch.setattr(capi, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        capi.lib()


def test_bench_headline_is_one_short_json_line():
    """bench.py's last stdout line is the headline alone: it parses as JSON,
    carries the contract's keys and stays within the size the driver reads
    whole, however many per-op rows the run measured (those go to stderr)."""
    import json
    import bench
    roofline = {"bound": "hbm", "achieved": 5800.0, "peak": 8000.0, "unit": "GB/s", "frac": 0.725,
                "traffic": 104882304, "kernel": "k" * 80, "launch": "l" * 120, "traffic_note": "t" * 300}
    cpu = {"value": 14.1, "unit": "GB/s", "cores": 16, "kind": "port", "sample": "s" * 400}
    line = bench.headline(value=4974.1, step_s=55.3e-6, steps=50, warmup=10, batch=32, launches=6,
                          step_bytes=275256576, nrot=3, roofline=roofline, cpu=cpu, op_rows=120)
    text = json.dumps(line)
    assert "\n" not in text and len(text) <= bench.HEADLINE_MAX_BYTES
    parsed = json.loads(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "dtype", "config",
                "pct_peak", "roofline", "cpu_baseline", "higher_is_better", "scaling", "vs_baseline", "data"):
        assert key in parsed, key
    assert "ops" not in parsed and parsed["roofline"]["frac"] == 0.725
    # over-long free text is shortened, never an error at the end of a run
    cpu["sample"] = "s" * 10000
    line = bench.headline(value=4974.1, step_s=55.3e-6, steps=50, warmup=10, batch=32, launches=6,
                          step_bytes=275256576, nrot=3, roofline=roofline, cpu=cpu, op_rows=120)
    assert len(json.dumps(line)) <= bench.HEADLINE_MAX_BYTES and line["cpu_baseline"]["value"] == 14.1


def test_bench_sweep_fit_recovers_a_line():
    """The size-sweep fit returns the floor and bandwidth of points lying on
    t = t0 + bytes / BW, and reports how far the worst point sits off it."""
    import bench
    pts = [(b, 1.6e-6 + b / 6.2e12) for b in (13e6, 26e6, 52e6, 105e6, 210e6, 315e6)]
    t0, bw, worst = bench.fit_line(pts)
    assert abs(t0 - 1.6) < 1e-9 and abs(bw - 6200.0) < 1e-6 and worst < 1e-12
    pts[0] = (pts[0][0], pts[0][1] * 1.1)
    assert bench.fit_line(pts)[2] > 0.05

"""PrivateUse1 ("npu") device backend on one MI355X (HIP device 0).

Drop-in for the reference's ``import thin_backend`` (thin_backend/__init__.py:
loads libthin_backend.so, renames PrivateUse1 to "npu", registers the device
module).  Every operator of the backend runs a hand-written gfx950 kernel
through libthin_hip.so; nothing falls back to the CPU.

The flow libraries keep the reference's file names next to this file:
libflow_ops.so, libconv_flow.so, libselection_flow.so, libthin_blocked.so,
libbmm_flow.so, libdepthwise_flow.so (load them with torch.ops.load_library).
"""
import os
from pathlib import Path
from types import SimpleNamespace

os.environ["TORCH_DEVICE_BACKEND_AUTOLOAD"] = "0"
import torch  # noqa: E402  (torch first: the libraries share its HIP runtime)

_HERE = Path(__file__).resolve().parent
_LIB = _HERE / "libthin_backend.so"
if not _LIB.exists():
    raise ImportError(f"{_LIB} is not built; run python -m thintnpu_amd.build")
torch.ops.load_library(str(_LIB))
torch.utils.rename_privateuse1_backend("npu")


def _device_count() -> int:
    return 1


def synchronize(device=None) -> None:
    """Wait for the calling thread's NPU stream."""
    torch.ops.thin_backend.synchronize()


torch._register_device_module("npu", SimpleNamespace(
    is_available=lambda: True,
    device_count=_device_count,
    current_device=lambda: 0,
    _is_in_bad_fork=lambda: False,
    manual_seed_all=lambda seed: None,
    _lazy_init=lambda: None,
    synchronize=synchronize,
    empty_cache=lambda: torch.ops.thin_backend.empty_cache(),
))
torch.utils.generate_methods_for_privateuse1_backend()

FLOW_LIBRARIES = ("libflow_ops.so", "libconv_flow.so", "libselection_flow.so", "libthin_blocked.so",
                  "libbmm_flow.so", "libdepthwise_flow.so")


def load_flow_libraries() -> None:
    """Load every flow library of this directory (idempotent)."""
    for name in FLOW_LIBRARIES:
        torch.ops.load_library(str(_HERE / name))

"""The frozen-region guard on the CPU: every drift a captured graph cannot see
raises ValueError with the contract's message (region_guard.cpp:119-184 in the
reference).  The Guard itself is device-agnostic, so CPU modules exercise it;
RegionContract's fp16-npu parameter rule is covered on the GPU."""
import types

import pytest
import torch
import torch.nn as nn

import thin_backend  # noqa: F401
from region_contract import ATTRIBUTES, RegionContract
from thin_backend._region_guard import Guard


def model():
    torch.manual_seed(0)
    m = nn.Sequential(nn.Conv2d(3, 8, 3, padding=1), nn.SiLU(), nn.Upsample(scale_factor=2.0))
    m.register_buffer("anchors", torch.zeros(4))
    for p in m.parameters():
        p.requires_grad_(False)
    return m.eval()


def guard(m, ignored=()):
    return Guard(list(m.modules()), set(ignored), ATTRIBUTES)


def test_unchanged_region_validates():
    m = model()
    g = guard(m)
    for _ in range(3):
        g.validate()


def mutations():
    def class_forward(m):
        original = nn.SiLU.forward
        nn.SiLU.forward = lambda self, x: x
        return lambda: setattr(nn.SiLU, "forward", original)

    def global_hook(m):
        handle = nn.modules.module.register_module_forward_hook(lambda *a: None)
        return handle.remove

    def swap_dict(m):
        m[1].__dict__ = dict(m[1].__dict__)

    return {
        "Region is inference-only": lambda m: m.train(),
        "Region hooks changed": lambda m: m[0].register_forward_hook(lambda *a: None),
        "Region child identity changed": lambda m: m.__setitem__(1, nn.SiLU()),
        "Region children changed": lambda m: m.append(nn.Identity()),
        "Region forward changed": lambda m: setattr(m[2], "forward", lambda x: x),
        "Region operator configuration changed": lambda m: setattr(m[0], "stride", (2, 2)),
        "Region parameter/prepack version or gradient mode changed": lambda m: m[0].weight.add_(1),
        "Region parameter/prepack identity changed": lambda m: setattr(m[0], "bias", nn.Parameter(
            m[0].bias.detach().clone(), requires_grad=False)),
        "Region parameter/buffer set changed": lambda m: m[0].register_buffer("extra", torch.zeros(1)),
        "Module class forward changed": class_forward,
        "Global module hooks are unsupported": global_hook,
        "Region module class changed": lambda m: setattr(m[1], "__class__", nn.GELU),
        "Region module dictionary changed": swap_dict,
        "Region attribute removed": lambda m: delattr(m[2], "_forward_hooks"),
    }


@pytest.mark.parametrize("message", list(mutations()))
def test_drift_is_rejected(message):
    m = model()
    g = guard(m)
    undo = mutations()[message](m)
    try:
        with pytest.raises(ValueError, match=message.replace("(", r"\(").replace(")", r"\)")):
            g.validate()
    finally:
        if isinstance(undo, (types.FunctionType, types.MethodType)):
            undo()


def test_gradient_mode_and_ignored_forward():
    m = model()
    g = guard(m, ignored=(m[2],))
    m[2].forward = lambda x: x          # the pilot swaps this forward itself
    g.validate()
    m[0].weight.requires_grad_(True)
    with pytest.raises(ValueError, match="gradient mode"):
        g.validate()


def test_contract_rejects_cpu_and_inference_tensors():
    with pytest.raises(ValueError, match="Expected fixed FP16 NPU inference parameters"):
        RegionContract((model(),))
    m = nn.Identity()
    with torch.inference_mode():
        m.register_buffer("frozen", torch.zeros(2))
    with pytest.raises(ValueError, match="no_grad"):
        RegionContract((m,))


def test_drifts_are_reported_in_contract_order():
    """When several drifts coexist, the first in the contract's order is the
    one reported: global hooks, then class forwards, then per module its class,
    __dict__, training, hooks, children, forward, attributes and tensors; and a
    drift in an earlier module before any drift in a later one."""
    m = model()
    g = guard(m)
    m.train()                                            # every module: training
    m[0].register_forward_hook(lambda *a: None)          # module 1: hooks
    with pytest.raises(ValueError, match="Region is inference-only"):
        g.validate()
    m.eval()
    with pytest.raises(ValueError, match="Region hooks changed"):
        g.validate()

    m = model()
    g = guard(m)
    m[2].forward = lambda x: x                           # module 3: forward
    m[1].inplace = True                                  # module 2: attribute
    with pytest.raises(ValueError, match="Region operator configuration changed"):
        g.validate()
    m[1].inplace = False
    with pytest.raises(ValueError, match="Region forward changed"):
        g.validate()

    m = model()
    g = guard(m)
    m[0].weight.add_(1)                                  # module 1: tensor version
    m[0].stride = (2, 2)                                 # module 1: attribute
    original = nn.Upsample.forward
    nn.Upsample.forward = lambda self, x: x              # a class forward
    handle = nn.modules.module.register_module_forward_hook(lambda *a: None)
    try:
        with pytest.raises(ValueError, match="Global module hooks are unsupported"):
            g.validate()
        handle.remove()
        with pytest.raises(ValueError, match="Module class forward changed"):
            g.validate()
    finally:
        handle.remove()
        nn.Upsample.forward = original
    with pytest.raises(ValueError, match="Region operator configuration changed"):
        g.validate()
    m[0].stride = (1, 1)
    with pytest.raises(ValueError, match="version or gradient mode"):
        g.validate()


def test_construction_errors():
    """Snapshot-time contract: a non-method forward, a non-tensor slot and a
    region that requires grad are rejected when the Guard is built."""
    m = model()
    m[1].forward = 3                                     # not a bound method
    with pytest.raises(ValueError, match="Expected a bound module forward"):
        guard(m)
    m = model()
    m[0]._parameters["odd"] = 3
    with pytest.raises(TypeError, match="Expected a Tensor or None"):
        guard(m)
    m = model()
    m[0].bias.requires_grad_(True)
    with pytest.raises(ValueError, match="gradient mode"):
        guard(m)
    m = model()
    m[0].bias = None                                     # a None slot is frozen as None
    g = guard(m)
    g.validate()
    m[0].bias = nn.Parameter(torch.zeros(8), requires_grad=False)
    with pytest.raises(ValueError, match="identity changed"):
        g.validate()

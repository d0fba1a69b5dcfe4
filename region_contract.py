"""RegionContract: the frozen-state contract a FrozenGraph pilot validates.

Same API as the reference's region_contract.py:5-28.  Construction checks that
every parameter and buffer of the region is a fixed fp16 ``npu`` inference
tensor with a version counter (prepared under ``no_grad()``, not
``inference_mode()``), then hands the modules to the native ``Guard``
(thintnpu_amd/csrc/torch/region_guard.cpp), whose ``validate()`` raises
ValueError on any drift: module class/dict, training mode, hooks, children,
forward bindings (except ``ignored_forward`` modules, whose forward the pilot
swaps itself), the operator attributes below, and parameter/buffer identity,
version, storage, shape, dtype and device.
"""
import torch

import thin_backend  # noqa: F401  (the npu device and the guard extension live there)
from thin_backend._region_guard import Guard

# Operator-configuration attributes frozen by the guard (the reference's list:
# nn.Conv2d / Upsample / MaxPool2d, Ultralytics Bottleneck / C2f / Attention /
# Detect fields, and the attributes the blocked rewrite sets).
ATTRIBUTES = ('in_channels', 'out_channels', 'kernel_size', 'stride', 'padding', 'padding_mode',
              'dilation', 'groups', 'add', 'c', 'inplace', 'scale_factor', 'mode',
              'align_corners', 'size', 'ceil_mode', 'return_indices',
              'num_heads', 'head_dim', 'key_dim', 'scale', 'shortcut', 'n', '_thin_attention_prescale',
              'nl', 'na', 'no', 'nc', 'export', 'reg_max', 'end2end', '_thin_strides',
              'max_det', 'agnostic_nms', 'xyxy')


class RegionContract:
    attributes = ATTRIBUTES

    def __init__(self, roots, ignored_forward=()):
        modules = [m for root in roots for m in root.modules()]
        for module in modules:
            for tensor in (*module._parameters.values(), *module._buffers.values()):
                if tensor is None:
                    continue
                try:
                    tensor._version
                except RuntimeError as error:
                    raise ValueError('Prepare versioned parameters under no_grad(), not inference_mode()') from error
                if tensor.requires_grad or tensor.dtype != torch.float16 or tensor.device.type != 'npu':
                    raise ValueError('Expected fixed FP16 NPU inference parameters')
        self.guard = Guard(modules, set(ignored_forward), self.attributes)

    def validate(self):
        self.guard.validate()

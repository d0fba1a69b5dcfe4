"""RegionContract: the frozen-state contract a FrozenGraph pilot validates.

The drop-in for the reference's region_contract.py:5-28. It has the same
constructor `RegionContract(roots, ignored_forward=())`, the same `attributes`
table and the same `validate()`. Both halves are native
(thintnpu_amd/csrc/torch/region_guard.cpp -> thin_backend/_region_guard*.so):

* `require_frozen_fp16` admits the region. Every parameter and buffer must be
  a version-counted (no_grad, not inference_mode) fp16 npu tensor without
  gradient. Anything else raises ValueError.
* `Guard` snapshots every module of the region. Its `validate()` raises
  ValueError on any drift a captured graph could not see:
  - class, `__dict__`, training mode, hooks, children;
  - forward bindings, except the modules in `ignored_forward`, whose forward
    the pilot swaps itself;
  - the operator attributes below;
  - parameter and buffer identity, version, storage and metadata.
"""
import thin_backend  # noqa: F401  (loads the npu device the parameters live on)
from thin_backend._region_guard import Guard, require_frozen_fp16

# Operator-configuration attributes the guard freezes. Pilots and their tests
# key on this table: nn.Conv2d / Upsample / MaxPool2d fields, Ultralytics
# Bottleneck / C2f / Attention / Detect fields, and the attributes the blocked
# rewrite sets.
ATTRIBUTES = ('in_channels', 'out_channels', 'kernel_size', 'stride', 'padding', 'padding_mode',
              'dilation', 'groups', 'add', 'c', 'inplace', 'scale_factor', 'mode',
              'align_corners', 'size', 'ceil_mode', 'return_indices',
              'num_heads', 'head_dim', 'key_dim', 'scale', 'shortcut', 'n', '_thin_attention_prescale',
              'nl', 'na', 'no', 'nc', 'export', 'reg_max', 'end2end', '_thin_strides',
              'max_det', 'agnostic_nms', 'xyxy')


class RegionContract:
    attributes = ATTRIBUTES

    def __init__(self, roots, ignored_forward=()):
        region = [module for root in roots for module in root.modules()]
        require_frozen_fp16(region)
        self.guard = Guard(region, set(ignored_forward), self.attributes)

    def validate(self):
        self.guard.validate()

// Host helpers of libthin_hip.so: error text, descriptor checks, coalescing.
#include "common.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace thin {

static thread_local char g_error[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int dtype_size(int32_t dtype) {
  switch (dtype) {
    case THIN_F16: return 2;
    case THIN_BF16: return 2;
    case THIN_I16: return 2;
    case THIN_F32: return 4;
    case THIN_I32: return 4;
    case THIN_I64: return 8;
    case THIN_F64: return 8;
    case THIN_U8: return 1;
    default: return 0;
  }
}

const char* dtype_name(int32_t dtype) {
  switch (dtype) {
    case THIN_F16: return "float16";
    case THIN_BF16: return "bfloat16";
    case THIN_I16: return "int16";
    case THIN_F32: return "float32";
    case THIN_I32: return "int32";
    case THIN_I64: return "int64";
    case THIN_F64: return "float64";
    case THIN_U8: return "uint8";
    default: return "unknown";
  }
}

int64_t numel(const thin_desc* d) {
  int64_t n = 1;
  for (int i = 0; i < d->rank; ++i) n *= d->sizes[i];
  return n;
}

bool desc_valid(const thin_desc* d) {
  if (!d || d->rank < 0 || d->rank > kMaxDims || dtype_size(d->dtype) == 0) return false;
  for (int i = 0; i < d->rank; ++i)
    if (d->sizes[i] < 0 || d->strides[i] < 0) return false;
  return numel(d) == 0 || d->data != nullptr;
}

bool same_sizes(const thin_desc* a, const thin_desc* b) {
  if (a->rank != b->rank) return false;
  for (int i = 0; i < a->rank; ++i)
    if (a->sizes[i] != b->sizes[i]) return false;
  return true;
}

bool is_contiguous(const thin_desc* d) {
  int64_t expect = 1;
  for (int i = d->rank - 1; i >= 0; --i) {
    if (d->sizes[i] == 1) continue;
    if (d->strides[i] != expect) return false;
    expect *= d->sizes[i];
  }
  return true;
}

Coalesced coalesce(const thin_desc* const* ops, int nops) {
  Coalesced c;
  c.nd = 0;
  const thin_desc* ref = ops[0];
  for (int d = 0; d < ref->rank; ++d) {
    int64_t n = ref->sizes[d];
    if (n == 1) continue;
    bool merge = c.nd > 0;
    for (int k = 0; merge && k < nops; ++k)
      merge = c.stride[k][c.nd - 1] == ops[k]->strides[d] * n;
    if (merge) {
      c.size[c.nd - 1] *= n;
      for (int k = 0; k < nops; ++k) c.stride[k][c.nd - 1] = ops[k]->strides[d];
    } else {
      c.size[c.nd] = n;
      for (int k = 0; k < nops; ++k) c.stride[k][c.nd] = ops[k]->strides[d];
      ++c.nd;
    }
  }
  if (c.nd == 0) {  // a single element
    c.nd = 1;
    c.size[0] = 1;
    for (int k = 0; k < nops; ++k) c.stride[k][0] = 1;
  }
  return c;
}

uint32_t grid_for(uint64_t units, uint32_t threads, uint32_t per_thread, uint32_t max_blocks) {
  uint64_t per_block = (uint64_t)threads * per_thread;
  uint64_t blocks = (units + per_block - 1) / per_block;
  if (blocks < 1) blocks = 1;
  if (blocks > max_blocks) blocks = max_blocks;
  return (uint32_t)blocks;
}

}  // namespace thin

extern "C" const char* thin_last_error(void) { return thin::g_error; }

extern "C" const char* thin_version(void) { return "thin-hip 0.1 gfx950"; }

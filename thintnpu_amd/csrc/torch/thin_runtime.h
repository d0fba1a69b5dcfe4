// Runtime shared by the PrivateUse1 ("npu") libraries: one logical device
// (HIP device 0), a HIP stream per host thread, a caching allocator, graph
// capture state and the glue between at::Tensor and the thin_hip C ABI.
#pragma once

#include <ATen/ATen.h>
#include <hip/hip_runtime_api.h>

#include "thin_hip.h"

namespace thin_rt {

constexpr auto kDevice = c10::DeviceType::PrivateUse1;

// HIP device 0 made current; rejects any other logical device
// (backend.cpp:32-35 exposes exactly logical NPU 0).
void select(c10::Device d);
void select();

// The calling thread's stream (created on first use, default priority).
hipStream_t stream();

// True while a RuntimeGraph captures on this thread.
bool capturing();

// Waits for the calling thread's stream unless it is capturing
// (backend.cpp:46).
void sync();

// Called after every eager launch: synchronizes the thread's stream (the
// reference's eager semantics) unless THIN_ASYNC=1 (one host thread only).
void after_launch();

// HIP error -> c10::Error.
void hip_check(hipError_t e, const char* what);

// thin_status -> c10::Error carrying thin_last_error().
void check(thin_status s, const char* what);

// Descriptor of a device tensor (storage offset folded into the pointer).
thin_desc desc(const at::Tensor& t);

// Inference-only device tensor check used by every op (ops.cpp:30-32).
void inference(const at::Tensor& x, const char* what);

// Device allocation through the caching allocator (workspace for ops).
at::Tensor empty_bytes(int64_t bytes);

at::Tensor& copy_(at::Tensor& dst, const at::Tensor& src, bool non_blocking);

// The value a 0-d CPU operand `s` takes in a binary op on a `dtype` tensor:
// converted to dtype first, as the reference converts it (ops.cpp:466-467).
// THIN_SCALAR_OPMATH=1 returns it unrounded instead; thin_binary_scalar then
// applies PyTorch CPU's rule (rounded to dtype for add/sub, fp32 for mul/div).
double scalar_operand(const at::Tensor& s, at::ScalarType dtype);

}  // namespace thin_rt

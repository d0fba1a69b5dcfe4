// PrivateUse1 runtime on HIP: device guard, per-thread stream, caching
// allocator (graph-retained capture allocations), empty/copy_/views, the
// host-computed constants (arange/fill_/item) and RuntimeGraph on hipGraph.
//
// Serves the reference runtime's surface (backend.cpp:32-206,312-361;
// graph_capture.h:7-24; decode.cpp:6-34; ops.cpp:32-78): one logical device,
// one stream per host thread, eager ops that have finished when they return
// (THIN_ASYNC=1 opts a single-threaded caller out of the per-op
// synchronize), and capture-time memory held until the graph closes.  Freed
// memory is cached per stream instead of being returned with a synchronizing
// free.
#include "thin_runtime.h"

#include <ATen/EmptyTensor.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/native/Resize.h>
#include <ATen/ops/as_strided_native.h>
#include <ATen/ops/view_native.h>
#include <ATen/ops/_reshape_alias_native.h>
#include <ATen/ops/split_native.h>
#include <ATen/ops/split_with_sizes_native.h>
#include <c10/core/Allocator.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>
#include <torch/custom_class.h>
#include <torch/library.h>

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace thin_rt {

void hip_check(hipError_t e, const char* what) {
  TORCH_CHECK(e == hipSuccess, what, " failed: ", hipGetErrorString(e));
}

void check(thin_status s, const char* what) {
  TORCH_CHECK(s == THIN_OK, what, ": ", thin_last_error());
}

void select() { hip_check(hipSetDevice(0), "hipSetDevice"); }

void select(c10::Device d) {
  TORCH_CHECK(d.type() == kDevice && (d.index() == -1 || d.index() == 0), "Only logical NPU 0 is exposed");
  select();
}

// Memory recorded while a RuntimeGraph captures (graph_capture.h:7-24): device
// blocks allocated or freed during capture stay with the graph until close().
struct GraphState {
  std::vector<void*> retained;  // freed by their tensors while the graph lives
  std::vector<void*> host;      // pinned staging of host->device copies
  bool alive = true;
};

thread_local GraphState* g_capture = nullptr;

bool capturing() { return g_capture != nullptr; }

// Eager ops synchronize their stream after each launch by default, as the
// reference's eager ops do (backend.cpp:46).  When an op returns its kernels
// have finished, so memory a host thread releases is never still read by
// another thread's stream, and the caching allocator may hand it out again at
// once.  THIN_ASYNC=1 leaves eager launches asynchronous.  That mode serves one
// host thread: its single stream orders every reuse of a block.  A second
// host thread that touches the device then fails loudly instead of racing.
static bool eager_async() {
  static const bool on = [] {
    const char* v = std::getenv("THIN_ASYNC");
    return v && std::strcmp(v, "1") == 0;
  }();
  return on;
}

static std::atomic<int> g_thread_streams{0};

hipStream_t stream() {
  thread_local hipStream_t s = [] {
    const int n = ++g_thread_streams;
    TORCH_CHECK(!eager_async() || n == 1,
                "THIN_ASYNC=1 allows one host thread on the NPU; unset it for multi-threaded use");
    select();
    hipStream_t p = nullptr;
    hip_check(hipStreamCreate(&p), "hipStreamCreate");
    return p;
  }();
  return s;
}

void sync() {
  if (!capturing()) hip_check(hipStreamSynchronize(stream()), "hipStreamSynchronize");
}

void after_launch() {
  if (!eager_async()) sync();
}

thin_desc desc(const at::Tensor& t) {
  thin_desc d;
  std::memset(&d, 0, sizeof d);
  TORCH_CHECK(t.dim() <= THIN_MAX_DIMS, "thin ops support up to ", THIN_MAX_DIMS, " dims");
  d.data = t.numel() ? const_cast<void*>(t.const_data_ptr()) : nullptr;
  switch (t.scalar_type()) {
    case at::kHalf: d.dtype = THIN_F16; break;
    case at::kFloat: d.dtype = THIN_F32; break;
    case at::kLong: d.dtype = THIN_I64; break;
    case at::kInt: d.dtype = THIN_I32; break;
    case at::kShort: d.dtype = THIN_I16; break;
    case at::kByte: case at::kChar: case at::kBool: d.dtype = THIN_U8; break;
    case at::kDouble: d.dtype = THIN_F64; break;
    case at::kBFloat16: d.dtype = THIN_BF16; break;
    default: TORCH_CHECK(false, "thin ops do not support dtype ", t.scalar_type());
  }
  d.rank = (int32_t)t.dim();
  for (int64_t i = 0; i < t.dim(); ++i) {
    d.sizes[i] = t.size(i);
    d.strides[i] = t.stride(i);
  }
  return d;
}

void inference(const at::Tensor& x, const char* what) {
  TORCH_CHECK(x.device().type() == kDevice && !x.requires_grad(), what,
              " requires inference-only NPU tensors");
}

// ------------------------------------------------------------------ allocator

namespace {

struct Block {
  size_t size;
  hipStream_t stream;
  GraphState* owner;
};

size_t round_size(size_t n) {
  if (n <= ((size_t)1 << 20)) return (n + 511) & ~(size_t)511;
  return (n + ((size_t)2 << 20) - 1) & ~(((size_t)2 << 20) - 1);
}

// Caching allocator.  A freed block returns to the free list of the stream it
// was allocated on and is reused only by later allocations on that stream, so
// reuse is ordered after every kernel that stream enqueued with it.  Work of
// other streams on the block has finished by the time it is released: eager
// ops complete before they return (after_launch; staging and resize copies
// included), and with THIN_ASYNC=1 there is only one stream.  Graph replays
// are the exception: they only enqueue.  A block a replay touches is either
// graph-owned (held until close(), which synchronizes) or state the caller
// keeps alive while the graph lives (parameters, the captured input); when
// the graph's own thread frees such a block, it returns to the graph's
// stream, whose later work is ordered after the replay.
class Pool {
 public:
  void* alloc(size_t n) {
    if (!n) return nullptr;
    const size_t sz = round_size(n);
    hipStream_t s = stream();
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = free_.find({s, sz});
    if (it != free_.end() && !it->second.empty()) {
      void* p = it->second.back();
      it->second.pop_back();
      live_[p].owner = g_capture;
      return p;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess && !capturing()) {
      (void)hipGetLastError();
      release_cached_locked();
      e = hipMalloc(&p, sz);
    }
    TORCH_CHECK(e == hipSuccess, "NPU allocation of ", sz, " bytes failed: ", hipGetErrorString(e));
    live_[p] = Block{sz, s, g_capture};
    return p;
  }

  void release(void* p) {
    if (!p) return;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = live_.find(p);
    if (it == live_.end()) return;
    Block& b = it->second;
    if (g_capture) {  // freed while this thread captures: graph kernels may use it
      b.owner = g_capture;
      g_capture->retained.push_back(p);
      return;
    }
    if (b.owner && b.owner->alive) {
      b.owner->retained.push_back(p);
      return;
    }
    b.owner = nullptr;
    free_[{b.stream, b.size}].push_back(p);
  }

  // RuntimeGraph::close after synchronizing its stream.
  void graph_closed(GraphState* g) {
    std::lock_guard<std::mutex> lock(mutex_);
    for (void* p : g->retained) {
      Block& b = live_[p];
      b.owner = nullptr;
      free_[{b.stream, b.size}].push_back(p);
    }
    g->retained.clear();
    for (auto& kv : live_)
      if (kv.second.owner == g) kv.second.owner = nullptr;
    g->alive = false;
  }

  void empty_cache() {
    if (capturing()) return;  // no device-wide synchronize inside a capture
    std::lock_guard<std::mutex> lock(mutex_);
    release_cached_locked();
  }

  size_t cached_bytes() {
    std::lock_guard<std::mutex> lock(mutex_);
    size_t n = 0;
    for (auto& kv : free_) n += kv.first.second * kv.second.size();
    return n;
  }

 private:
  void release_cached_locked() {
    if (free_.empty()) return;
    (void)hipDeviceSynchronize();
    for (auto& kv : free_)
      for (void* p : kv.second) {
        live_.erase(p);
        (void)hipFree(p);
      }
    free_.clear();
  }

  std::mutex mutex_;
  std::unordered_map<void*, Block> live_;
  std::map<std::pair<hipStream_t, size_t>, std::vector<void*>> free_;
};

Pool& pool() {
  static Pool* p = new Pool();  // intentionally leaked: outlives static tensors
  return *p;
}

void release_ptr(void* p) { pool().release(p); }

struct Allocator final : c10::Allocator {
  c10::DataPtr allocate(size_t n) override {
    select();
    void* p = pool().alloc(n);
    return {p, p, &release_ptr, c10::Device(kDevice, 0)};
  }
  c10::DeleterFnPtr raw_deleter() const override { return &release_ptr; }
  void copy_data(void* dst, const void* src, std::size_t n) const override {
    if (n) hip_check(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, stream()), "hipMemcpyAsync");
  }
};

Allocator g_allocator;

// ------------------------------------------------------------------ guard

struct Guard final : c10::impl::DeviceGuardImplInterface {
  c10::DeviceType type() const override { return kDevice; }
  c10::Device getDevice() const override { return c10::Device(kDevice, 0); }
  c10::Device exchangeDevice(c10::Device d) const override {
    select(d);
    return getDevice();
  }
  void setDevice(c10::Device d) const override { select(d); }
  void uncheckedSetDevice(c10::Device) const noexcept override { (void)hipSetDevice(0); }
  c10::Stream getStream(c10::Device d) const override {
    select(d);
    (void)stream();
    return c10::Stream(c10::Stream::DEFAULT, getDevice());
  }
  c10::Stream getDefaultStream(c10::Device d) const override { return getStream(d); }
  c10::Stream exchangeStream(c10::Stream s) const override {
    TORCH_CHECK(s.id() == 0, "Only the default stream is supported");
    return getStream(s.device());
  }
  c10::DeviceIndex deviceCount() const noexcept override {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0 ? 1 : 0;
  }
  void synchronizeStream(const c10::Stream&) const override { sync(); }
  void synchronizeDevice(c10::DeviceIndex) const override {
    if (!capturing()) hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  }
};

// ------------------------------------------------------------------ factories

void validate_options(std::optional<at::Layout> layout, std::optional<c10::Device> device,
                      std::optional<bool> pin) {
  TORCH_CHECK(!layout || *layout == at::kStrided, "Only strided layout is supported");
  TORCH_CHECK(!pin.value_or(false), "Pinned allocation is not implemented");
  select(device.value_or(c10::Device(kDevice, 0)));
}

at::Tensor empty(c10::SymIntArrayRef size, std::optional<at::ScalarType> dtype, std::optional<at::Layout> layout,
                 std::optional<c10::Device> device, std::optional<bool> pin,
                 std::optional<c10::MemoryFormat> format) {
  validate_options(layout, device, pin);
  return at::detail::empty_generic_symint(size, &g_allocator, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1),
                                          dtype.value_or(at::kFloat), format);
}

at::Tensor empty_strided(c10::SymIntArrayRef size, c10::SymIntArrayRef stride, std::optional<at::ScalarType> dtype,
                         std::optional<at::Layout> layout, std::optional<c10::Device> device,
                         std::optional<bool> pin) {
  validate_options(layout, device, pin);
  return at::detail::empty_strided_symint_generic(size, stride, &g_allocator,
                                                  c10::DispatchKeySet(c10::DispatchKey::PrivateUse1),
                                                  dtype.value_or(at::kFloat));
}

// resize_ for out= variants: grows the storage through the caching allocator.
const at::Tensor& resize_(const at::Tensor& self, c10::SymIntArrayRef size,
                          std::optional<c10::MemoryFormat> format) {
  TORCH_CHECK(!format || *format == c10::MemoryFormat::Contiguous, "thin resize_ supports contiguous format only");
  auto* impl = self.unsafeGetTensorImpl();
  int64_t numel = 1;
  std::vector<int64_t> sizes;
  for (auto s : size) {
    sizes.push_back(s.expect_int());
    numel *= sizes.back();
  }
  const size_t needed = (size_t)(impl->storage_offset() + numel) * self.itemsize();
  if (needed > impl->storage().nbytes()) {
    c10::Storage fresh(c10::Storage::use_byte_size_t(), needed, g_allocator.allocate(needed), &g_allocator, true);
    const size_t old = impl->storage().nbytes();
    if (old && impl->storage().data())
      hip_check(hipMemcpyAsync(fresh.mutable_data(), impl->storage().data(), old, hipMemcpyDeviceToDevice, stream()),
                "hipMemcpyAsync");
    if (old) after_launch();  // the old storage may be released to another thread
    impl->set_storage_keep_dtype(std::move(fresh));
  }
  impl->set_sizes_contiguous(sizes);
  return self;
}

}  // namespace

at::Tensor empty_bytes(int64_t bytes) {
  return at::empty({std::max<int64_t>(bytes, 1)}, at::TensorOptions().dtype(at::kByte).device(kDevice, 0));
}

// ------------------------------------------------------------------ copy_
// aten::copy_ (ops.cpp:32-78): device<->device through the strided bit-copy
// kernel, host<->device through hipMemcpyAsync of dense staging buffers.
double scalar_operand(const at::Tensor& s, at::ScalarType dtype) {
  static const bool opmath = [] {
    const char* v = std::getenv("THIN_SCALAR_OPMATH");
    return v && std::string(v) == "1";
  }();
  return opmath ? s.item<double>() : s.to(dtype).item<double>();
}

at::Tensor& copy_(at::Tensor& dst, const at::Tensor& src_in, bool non_blocking) {
  (void)non_blocking;
  TORCH_CHECK(dst.scalar_type() == src_in.scalar_type(), "copy requires matching sizes and dtype");
  const bool dn = dst.device().type() == kDevice, sn = src_in.device().type() == kDevice;
  TORCH_CHECK((dn || dst.is_cpu()) && (sn || src_in.is_cpu()) && (dn || sn), "Unsupported copy devices");
  if (dst.is_same(src_in) || !dst.numel()) return dst;
  at::Tensor src = src_in.sizes() == dst.sizes() ? src_in : src_in.expand(dst.sizes());
  at::assert_no_internal_overlap(dst);
  at::assert_no_partial_overlap(dst, src);
  select();
  TORCH_CHECK(!capturing() || dn, "Device-to-host copy is not allowed during graph capture");
  if (dn && sn) {
    thin_desc s = desc(src), d = desc(dst);
    check(thin_copy(&s, &d, stream()), "thin copy_");
    after_launch();
    return dst;
  }
  if (dn) {  // host -> device
    at::Tensor host = src.contiguous();
    const bool direct = dst.is_contiguous();
    at::Tensor stage = direct ? dst : at::empty(dst.sizes(), dst.options());
    const size_t bytes = host.nbytes();
    const void* from = host.const_data_ptr();
    if (capturing()) {
      // Pageable uploads cannot be recorded; the graph owns a pinned copy.
      void* pinned = nullptr;
      hip_check(hipHostMalloc(&pinned, bytes, hipHostMallocDefault), "hipHostMalloc");
      std::memcpy(pinned, from, bytes);
      g_capture->host.push_back(pinned);
      from = pinned;
    }
    hip_check(hipMemcpyAsync(stage.data_ptr(), from, bytes, hipMemcpyHostToDevice, stream()), "hipMemcpyAsync");
    if (!capturing()) sync();  // the host buffer may be released after return
    if (!direct) {
      thin_desc s = desc(stage), d = desc(dst);
      check(thin_copy(&s, &d, stream()), "thin copy_");
      after_launch();  // dst may belong to another thread's stream
    }
    return dst;
  }
  // device -> host
  at::Tensor dev = src;
  if (!src.is_contiguous()) {
    dev = at::empty(src.sizes(), src.options().memory_format(c10::MemoryFormat::Contiguous));
    thin_desc s = desc(src), d = desc(dev);
    check(thin_copy(&s, &d, stream()), "thin copy_");
  }
  at::Tensor host = dst.is_contiguous() ? dst : at::empty(dst.sizes(), dst.options());
  hip_check(hipMemcpyAsync(host.data_ptr(), dev.const_data_ptr(), host.nbytes(), hipMemcpyDeviceToHost, stream()),
            "hipMemcpyAsync");
  hip_check(hipStreamSynchronize(stream()), "hipStreamSynchronize");
  if (!dst.is_contiguous()) dst.copy_(host);
  return dst;
}

// ------------------------------------------------------------------ host constants
// decode.cpp:6-34: arange computed on the CPU and uploaded; fill_ on the device.
namespace {

at::Tensor& arange_out(const at::Scalar& start, const at::Scalar& end, const at::Scalar& step, at::Tensor& out) {
  auto constant = at::arange(start, end, step, out.options().device(at::kCPU));
  if (out.sizes() != constant.sizes()) {
    auto replacement = at::empty(constant.sizes(), out.options());
    out.unsafeGetTensorImpl()->set_storage_keep_dtype(replacement.storage());
    out.unsafeGetTensorImpl()->set_storage_offset(0);
    out.unsafeGetTensorImpl()->set_sizes_contiguous(constant.sizes());
  }
  return copy_(out, constant, false);
}

at::Tensor& arange_end_out(const at::Scalar& end, at::Tensor& out) { return arange_out(0, end, 1, out); }

// fill_ / zero_ run the thin_fill kernel on the device (any strides; capture-safe).
at::Tensor& fill(at::Tensor& out, const at::Scalar& value) {
  if (!out.numel()) return out;
  select(out.device());
  thin_desc od = desc(out);
  const bool fp = at::isFloatingType(out.scalar_type());
  check(thin_fill(&od, fp ? value.toDouble() : 0.0, fp ? 0 : value.toLong(), stream()), "fill_");
  after_launch();
  return out;
}

at::Tensor& zero(at::Tensor& out) { return fill(out, 0); }

at::Scalar local_scalar(const at::Tensor& x) {
  TORCH_CHECK(x.numel() == 1, "_local_scalar_dense requires one element");
  auto host = at::empty(x.sizes(), x.options().device(at::kCPU));
  copy_(host, x, false);
  return host.item();
}

at::Tensor& copy_entry(at::Tensor& dst, const at::Tensor& src, bool non_blocking) {
  return copy_(dst, src, non_blocking);
}

// ------------------------------------------------------------------ RuntimeGraph
// thin_backend::RuntimeGraph (the reference's capture object, backend.cpp:62-113)
// on hipGraph.  One object records the creating thread's stream once and
// replays it:
//
//   kEmpty --begin()--> kRecording --end()--> kExecutable --replay()*--> ...
//   any phase --close()--> kClosed (idempotent)
//
// While recording, the allocator routes every block allocated or freed by
// this thread to the graph's GraphState, so memory the recorded kernels touch
// stays valid until close().  The executable is uploaded to the stream at
// end(), so the first replay pays no upload.  Every call must come from the
// creating thread, whose stream the graph is bound to.
//
// Replay dispatch.  hipGraphLaunch costs about 14 us of host time per call
// whatever the graph holds (1 to 3 kernel nodes measured alike on MI355X),
// while one hipLaunchKernel costs about 2.8 us.  A recording that is a
// straight chain of at most kDirectNodes plain kernel nodes (one root, each
// node with one successor, no memcpy/memset/host nodes, no `extra` argument
// blocks) is therefore replayed by launching its kernels in order on the
// graph's stream, from the parameters the recorded nodes hold (their argument
// arrays live as long as the recorded graph, which close() destroys).  The
// stream order of one chain is exactly the graph's dependency order.  Every
// other recording, and every recording when THIN_GRAPH_DIRECT=0, replays
// through hipGraphLaunch.
class RuntimeGraph : public torch::CustomClassHolder {
 public:
  enum class Phase { kEmpty, kRecording, kExecutable, kClosed };

  void begin() {
    require_owner();
    TORCH_CHECK(phase_ == Phase::kEmpty, "RuntimeGraph.begin: ", describe(),
                "; a RuntimeGraph records exactly once");
    TORCH_CHECK(!capturing(), "RuntimeGraph.begin: this thread is already recording another graph");
    sync();  // eager work enqueued before the recording must not be recorded
    hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    g_capture = memory_.get();
    phase_ = Phase::kRecording;
  }

  void end() {
    require_owner();
    TORCH_CHECK(phase_ == Phase::kRecording && g_capture == memory_.get(), "RuntimeGraph.end: ", describe(),
                ", not recording");
    hipGraph_t recorded = nullptr;
    const hipError_t e = hipStreamEndCapture(stream_, &recorded);
    g_capture = nullptr;
    phase_ = Phase::kExecutable;  // close() releases whatever was built, also on failure
    exec_.graph = recorded;
    hip_check(e, "hipStreamEndCapture");
    hip_check(hipGraphInstantiate(&exec_.exec, exec_.graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    hip_check(hipGraphUpload(exec_.exec, stream_), "hipGraphUpload");
    if (direct_enabled()) {
      exec_.chain = kernel_chain(exec_.graph);
      (void)hipGetLastError();  // a refused query only means: replay through hipGraphLaunch
    }
  }

  void replay() {
    require_owner();
    TORCH_CHECK(phase_ == Phase::kExecutable && exec_.exec, "RuntimeGraph.replay: ", describe(),
                ", nothing to replay");
    TORCH_CHECK(!capturing(), "RuntimeGraph.replay: cannot launch a graph while this thread records one");
    // Enqueue only, as the reference's replay does (backend.cpp:89-93).  The
    // graph's memory stays reserved until close(), which synchronizes; a D2H
    // copy or synchronize() on this thread waits for the replay.
    if (exec_.chain.empty()) {
      hip_check(hipGraphLaunch(exec_.exec, stream_), "hipGraphLaunch");
      return;
    }
    for (const hipKernelNodeParams& k : exec_.chain)
      hip_check(hipLaunchKernel(k.func, k.gridDim, k.blockDim, k.kernelParams, k.sharedMemBytes, stream_),
                "hipLaunchKernel (graph replay)");
  }

  // Whether replay() dispatches the recorded kernels itself (runtime helper
  // for tests and benchmarks; not part of the reference surface).
  bool direct() const { return !exec_.chain.empty(); }

  void close() {
    require_owner();
    if (phase_ == Phase::kClosed) return;
    if (phase_ == Phase::kRecording) {  // abandon the recording; nothing of it is kept
      hipGraph_t partial = nullptr;
      (void)hipStreamEndCapture(stream_, &partial);
      g_capture = nullptr;
      if (partial) (void)hipGraphDestroy(partial);
    }
    TORCH_CHECK(!capturing(), "RuntimeGraph.close: this thread is recording another graph");
    hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");  // last replay done
    exec_.destroy();
    pool().graph_closed(memory_.get());
    for (void* h : memory_->host) (void)hipHostFree(h);
    memory_->host.clear();
    phase_ = Phase::kClosed;
  }

  ~RuntimeGraph() override {
    if (phase_ == Phase::kClosed) return;
    try {
      close();
    } catch (const std::exception& error) {
      // The device may still use the graph's memory: keep every block it
      // holds out of the allocator for the rest of the process.
      std::fprintf(stderr, "RuntimeGraph: close in destructor failed, its memory stays reserved: %s\n",
                   error.what());
      (void)memory_.release();
    }
  }

 private:
  struct Executable {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<hipKernelNodeParams> chain;  // direct-dispatch form; empty: hipGraphLaunch
    void destroy() {
      chain.clear();
      if (exec) hip_check(hipGraphExecDestroy(exec), "hipGraphExecDestroy");
      exec = nullptr;
      if (graph) hip_check(hipGraphDestroy(graph), "hipGraphDestroy");
      graph = nullptr;
    }
  };

  static constexpr size_t kDirectNodes = 4;  // at 5+ nodes one hipGraphLaunch is cheaper

  static bool direct_enabled() {
    static const bool on = [] {
      const char* v = std::getenv("THIN_GRAPH_DIRECT");
      return !(v && std::strcmp(v, "0") == 0);
    }();
    return on;
  }

  // The recording's kernels in dependency order when it is a straight chain
  // of at most kDirectNodes plain kernel nodes; empty otherwise.
  static std::vector<hipKernelNodeParams> kernel_chain(hipGraph_t g) {
    std::vector<hipKernelNodeParams> out;
    size_t count = 0;
    if (hipGraphGetNodes(g, nullptr, &count) != hipSuccess || count == 0 || count > kDirectNodes) return {};
    size_t roots = 0;
    if (hipGraphGetRootNodes(g, nullptr, &roots) != hipSuccess || roots != 1) return {};
    hipGraphNode_t node = nullptr;
    if (hipGraphGetRootNodes(g, &node, &roots) != hipSuccess) return {};
    while (node) {
      hipGraphNodeType type;
      if (hipGraphNodeGetType(node, &type) != hipSuccess || type != hipGraphNodeTypeKernel) return {};
      size_t deps = 0;
      if (hipGraphNodeGetDependencies(node, nullptr, &deps) != hipSuccess || deps > 1) return {};
      hipKernelNodeParams k{};
      if (hipGraphKernelNodeGetParams(node, &k) != hipSuccess || !k.func || k.extra) return {};
      out.push_back(k);
      size_t next = 0;
      if (hipGraphNodeGetDependentNodes(node, nullptr, &next) != hipSuccess || next > 1) return {};
      hipGraphNode_t successor = nullptr;
      if (next == 1 && hipGraphNodeGetDependentNodes(node, &successor, &next) != hipSuccess) return {};
      node = successor;
      if (out.size() > count) return {};
    }
    if (out.size() != count) return {};
    return out;
  }

  // The graph is bound to the creating thread's stream.  The message is the
  // one callers of the reference key on ("creating thread/stream").
  void require_owner() const {
    TORCH_CHECK(std::this_thread::get_id() == owner_ && stream() == stream_,
                "RuntimeGraph must stay on its creating thread/stream");
  }

  const char* describe() const {
    switch (phase_) {
      case Phase::kEmpty: return "the graph is empty";
      case Phase::kRecording: return "the graph is recording";
      case Phase::kExecutable: return "the graph is already recorded";
      default: return "the graph is closed";
    }
  }

  const std::thread::id owner_ = std::this_thread::get_id();
  const hipStream_t stream_ = stream();
  std::unique_ptr<GraphState> memory_ = std::make_unique<GraphState>();
  Executable exec_;
  Phase phase_ = Phase::kEmpty;
};

void empty_cache() { pool().empty_cache(); }
int64_t cached_bytes() { return (int64_t)pool().cached_bytes(); }
void synchronize() { sync(); }

}  // namespace
}  // namespace thin_rt

C10_REGISTER_GUARD_IMPL(PrivateUse1, thin_rt::Guard);
REGISTER_ALLOCATOR(c10::DeviceType::PrivateUse1, &thin_rt::g_allocator);

TORCH_LIBRARY(thin_backend, m) {
  m.class_<thin_rt::RuntimeGraph>("RuntimeGraph")
      .def(torch::init<>())
      .def("begin", &thin_rt::RuntimeGraph::begin)
      .def("end", &thin_rt::RuntimeGraph::end)
      .def("replay", &thin_rt::RuntimeGraph::replay)
      .def("close", &thin_rt::RuntimeGraph::close)
      .def("direct", &thin_rt::RuntimeGraph::direct);
  // reference surface (backend.cpp:320-339); conv/maxpool/nms raise
  m.def("conv2d_prepare(Tensor w) -> Tensor");
  m.def("conv2d_prepared(Tensor x, Tensor w, Tensor packed, Tensor? bias, int stride, int pad, bool fp32_output=False, "
        "bool fused=False) -> Tensor");
  m.def("conv2d_fused(Tensor x, Tensor w, Tensor? bias, int stride, int pad, bool fp32_output=False, "
        "bool fused=True) -> Tensor");
  m.def("add(Tensor x, Tensor y) -> Tensor");
  m.def("sigmoid(Tensor x) -> Tensor");
  m.def("maxpool2d(Tensor x) -> Tensor");
  m.def("upsample_nearest2d(Tensor x) -> Tensor");
  m.def("conv2d(Tensor x, Tensor w, Tensor? bias=None, int stride=1, int pad=1, bool fp32_output=False) -> Tensor");
  m.def("nms(Tensor boxes, Tensor scores, float iou) -> Tensor");
  // runtime helpers of this backend
  m.def("synchronize() -> ()", &thin_rt::synchronize);
  m.def("empty_cache() -> ()", &thin_rt::empty_cache);
  m.def("cached_bytes() -> int", &thin_rt::cached_bytes);
}

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("empty.memory_format", TORCH_FN(thin_rt::empty));
  m.impl("empty_strided", TORCH_FN(thin_rt::empty_strided));
  m.impl("copy_", TORCH_FN(thin_rt::copy_entry));
  m.impl("resize_", TORCH_FN(thin_rt::resize_));
  m.impl("as_strided", TORCH_FN(at::native::as_strided_tensorimpl));
  m.impl("view", TORCH_FN(at::native::view));
  m.impl("_reshape_alias", TORCH_FN(at::native::_reshape_alias));
  m.impl("split.Tensor", TORCH_FN(at::native::split));
  m.impl("split_with_sizes", TORCH_FN(at::native::split_with_sizes));
  m.impl("arange.start_out", TORCH_FN(thin_rt::arange_out));
  m.impl("arange.out", TORCH_FN(thin_rt::arange_end_out));
  m.impl("fill_.Scalar", TORCH_FN(thin_rt::fill));
  m.impl("zero_", TORCH_FN(thin_rt::zero));
  m.impl("_local_scalar_dense", TORCH_FN(thin_rt::local_scalar));
}

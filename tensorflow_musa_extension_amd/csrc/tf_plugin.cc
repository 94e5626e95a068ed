// TensorFlow PluggableDevice adapter: the three entry points TensorFlow looks
// up in a pluggable device library (load_pluggable_device_library), built as
// libtfma_tf.so on top of the C ABI of libtfma.so.
//
//   SE_InitPlugin  - the StreamExecutor platform: device enumeration, memory,
//                    streams, events, timers, copies, host callbacks
//                    (replaces musa_ext/mu/musa_se_plugin.cc:1235-1297 and the
//                    SP_StreamExecutor table at :1166-1213);
//   TF_InitKernel  - kernels for the hot-path ops through TF_NewKernelBuilder,
//                    with the type constraints and HostMemory arguments of the
//                    reference's registrations
//                    (musa_ext/kernels/nn/musa_fused_batchnorm_op.cc:303-325,
//                    musa_ext/kernels/training/musa_applyadam_op.cc:645-682,
//                    musa_applyadam_mixed_op.cc:285-300), and the op
//                    definitions of the fused and grouped ops
//                    (musa_applyadam_mixed_op.cc:265-281,
//                    musa_ext/kernels/fusion/musa_shifted_affine_map_op.cc:108);
//                    the reference's own TF_InitKernel registers nothing
//                    (musa_ext/mu/kernel_register.cc:22-25);
//   TF_InitGraph   - the fusion / grouping rewrite as a Grappler plugin
//                    optimizer (the reference registers its pass in C++,
//                    musa_ext/mu/optimizer/musa_graph_optimizer.cc:6279).
//
// Device type "AMDGPU" (distinct from TensorFlow's built-in "GPU"), platform
// "AMDGPU_ROCM".  Every callback sets a TF_Status and never throws; kernels
// enqueue on the stream TensorFlow hands them and never synchronize the host.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "tf_c_api.h"
#include "tfma.h"

struct SP_Stream_st {
  hipStream_t stream;
  int device;
};
struct SP_Event_st {
  hipEvent_t event;
};
struct SP_Timer_st {
  hipEvent_t start;
  hipEvent_t stop;
};

namespace {

constexpr char kDeviceType[] = "AMDGPU";
constexpr char kPlatformName[] = "AMDGPU_ROCM";
constexpr char kVendor[] = "AMD";

// ---------------------------------------------------------------------------
// Status helpers.
// ---------------------------------------------------------------------------
void set_ok(TF_Status* s) { TF_SetStatus(s, TF_OK, ""); }

void set_error(TF_Status* s, TF_Code code, const char* fmt, ...)
    __attribute__((format(printf, 3, 4)));
void set_error(TF_Status* s, TF_Code code, const char* fmt, ...) {
  char buf[600];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  TF_SetStatus(s, code, buf);
}

bool hip_ok(hipError_t e, TF_Status* s, const char* what) {
  if (e == hipSuccess) {
    set_ok(s);
    return true;
  }
  set_error(s, TF_INTERNAL, "%s: %s", what, hipGetErrorString(e));
  return false;
}

// Makes the SP_Device's ordinal current on the calling thread (TensorFlow
// calls the plugin from many threads).
bool use_device(const SP_Device* d, TF_Status* s) {
  if (!d) {
    if (s) set_error(s, TF_INVALID_ARGUMENT, "null device");
    return false;
  }
  const hipError_t e = hipSetDevice(d->ordinal);
  if (e != hipSuccess) {
    if (s) set_error(s, TF_INTERNAL, "hipSetDevice(%d): %s", d->ordinal, hipGetErrorString(e));
    return false;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Platform and device.
// ---------------------------------------------------------------------------
struct DeviceInfo {
  std::string name;
  std::string pci_bus_id;
};

void get_device_count(const SP_Platform*, int* count, TF_Status* s) {
  TFMA_Status st;
  if (TFMA_GetDeviceCount(count, &st) != TFMA_OK) {
    set_error(s, TF_INTERNAL, "%s", st.message);
    return;
  }
  set_ok(s);  // no driver or no device: 0 devices and OK
}

void create_device(const SP_Platform*, SE_CreateDeviceParams* p, TF_Status* s) {
  if (!p || !p->device) {
    set_error(s, TF_INVALID_ARGUMENT, "create_device: null params or device");
    return;
  }
  if (p->struct_size < SE_CREATE_DEVICE_PARAMS_STRUCT_SIZE ||
      p->device->struct_size < SP_DEVICE_STRUCT_SIZE) {
    set_error(s, TF_INVALID_ARGUMENT, "create_device: struct_size too small");
    return;
  }
  SP_Device* d = p->device;
  d->struct_size = SP_DEVICE_STRUCT_SIZE;
  d->ordinal = p->ordinal;
  d->device_handle = reinterpret_cast<void*>(static_cast<intptr_t>(p->ordinal));
  d->device_vendor = kVendor;
  d->hardware_name = kPlatformName;
  d->pci_bus_id = nullptr;
  auto* info = new DeviceInfo();
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, p->ordinal) == hipSuccess) {
    info->name = prop.gcnArchName[0] ? prop.gcnArchName : prop.name;
    char bus[64] = {0};
    if (hipDeviceGetPCIBusId(bus, sizeof(bus), p->ordinal) == hipSuccess) info->pci_bus_id = bus;
  }
  if (!info->name.empty()) d->hardware_name = info->name.c_str();
  if (!info->pci_bus_id.empty()) d->pci_bus_id = info->pci_bus_id.c_str();
  d->ext = info;
  set_ok(s);
}

void destroy_device(const SP_Platform*, SP_Device* d) {
  if (!d) return;
  delete static_cast<DeviceInfo*>(d->ext);
  d->ext = nullptr;
  d->hardware_name = nullptr;
  d->pci_bus_id = nullptr;
}

int32_t get_numa_node(const SP_Device*) { return -1; }

int64_t get_memory_bandwidth(const SP_Device* d) {
  int khz = 0, bits = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeMemoryClockRate, d->ordinal) != hipSuccess ||
      hipDeviceGetAttribute(&bits, hipDeviceAttributeMemoryBusWidth, d->ordinal) != hipSuccess)
    return 0;
  // Double data rate: bytes/s = 2 * clock * bus width / 8.
  return static_cast<int64_t>(2) * khz * 1000 * (bits / 8);
}

double get_gflops(const SP_Device*) { return -1.0; }

void create_device_fns(const SP_Platform*, SE_CreateDeviceFnsParams* p, TF_Status* s) {
  if (!p || !p->device_fns) {
    set_error(s, TF_INVALID_ARGUMENT, "create_device_fns: null params");
    return;
  }
  SP_DeviceFns* f = p->device_fns;
  f->struct_size = SP_DEVICE_FNS_STRUCT_SIZE;
  f->get_numa_node = get_numa_node;
  f->get_memory_bandwidth = get_memory_bandwidth;
  f->get_gflops = get_gflops;
  set_ok(s);
}

void destroy_device_fns(const SP_Platform*, SP_DeviceFns*) {}

// ---------------------------------------------------------------------------
// Memory.  With use_bfc_allocator = 1 TensorFlow puts its BFC allocator on
// top of these, so allocate/deallocate see few, large requests.
// ---------------------------------------------------------------------------
struct AllocCounters {
  std::atomic<int64_t> num_allocs{0}, bytes_in_use{0}, peak{0}, largest{0};
};
AllocCounters g_alloc[64];

AllocCounters* counters(const SP_Device* d) {
  return (d && d->ordinal >= 0 && d->ordinal < 64) ? &g_alloc[d->ordinal] : nullptr;
}

void allocate(const SP_Device* d, uint64_t size, int64_t /*memory_space*/,
              SP_DeviceMemoryBase* mem) {
  mem->struct_size = SP_DEVICE_MEMORY_BASE_STRUCT_SIZE;
  mem->opaque = nullptr;
  mem->size = 0;
  if (!use_device(d, nullptr) || size == 0) return;
  void* p = nullptr;
  if (hipMalloc(&p, size) != hipSuccess) return;  // opaque stays null: TF sees the failure
  mem->opaque = p;
  mem->size = size;
  if (AllocCounters* c = counters(d)) {
    c->num_allocs++;
    const int64_t now = c->bytes_in_use += static_cast<int64_t>(size);
    int64_t pk = c->peak.load();
    while (now > pk && !c->peak.compare_exchange_weak(pk, now)) {
    }
    int64_t lg = c->largest.load();
    while (static_cast<int64_t>(size) > lg &&
           !c->largest.compare_exchange_weak(lg, static_cast<int64_t>(size))) {
    }
  }
}

void deallocate(const SP_Device* d, SP_DeviceMemoryBase* mem) {
  if (!mem || !mem->opaque) return;
  if (!use_device(d, nullptr)) return;
  (void)hipFree(mem->opaque);
  if (AllocCounters* c = counters(d)) c->bytes_in_use -= static_cast<int64_t>(mem->size);
  mem->opaque = nullptr;
  mem->size = 0;
}

void* host_memory_allocate(const SP_Device* d, uint64_t size) {
  if (!use_device(d, nullptr)) return nullptr;
  void* p = nullptr;
  return hipHostMalloc(&p, size, hipHostMallocDefault) == hipSuccess ? p : nullptr;
}

void host_memory_deallocate(const SP_Device* d, void* mem) {
  if (!mem || !use_device(d, nullptr)) return;
  (void)hipHostFree(mem);
}

void* unified_memory_allocate(const SP_Device* d, uint64_t bytes) {
  if (!use_device(d, nullptr)) return nullptr;
  void* p = nullptr;
  return hipMallocManaged(&p, bytes, hipMemAttachGlobal) == hipSuccess ? p : nullptr;
}

void unified_memory_deallocate(const SP_Device* d, void* p) {
  if (!p || !use_device(d, nullptr)) return;
  (void)hipFree(p);
}

TF_Bool get_allocator_stats(const SP_Device* d, SP_AllocatorStats* st) {
  AllocCounters* c = counters(d);
  if (!c || !st) return 0;
  st->struct_size = SP_ALLOCATORSTATS_STRUCT_SIZE;
  st->num_allocs = c->num_allocs.load();
  st->bytes_in_use = c->bytes_in_use.load();
  st->peak_bytes_in_use = c->peak.load();
  st->largest_alloc_size = c->largest.load();
  st->has_bytes_limit = 0;
  st->bytes_limit = 0;
  st->bytes_reserved = 0;
  st->peak_bytes_reserved = 0;
  st->has_bytes_reservable_limit = 0;
  st->bytes_reservable_limit = 0;
  st->largest_free_block_bytes = 0;
  return 1;
}

TF_Bool device_memory_usage(const SP_Device* d, int64_t* free_b, int64_t* total_b) {
  if (!use_device(d, nullptr)) return 0;
  size_t f = 0, t = 0;
  if (hipMemGetInfo(&f, &t) != hipSuccess) return 0;
  *free_b = static_cast<int64_t>(f);
  *total_b = static_cast<int64_t>(t);
  return 1;
}

// ---------------------------------------------------------------------------
// Streams and events (default priority; non-blocking with respect to the
// null stream, whose synchronous copies TensorFlow orders itself).
// ---------------------------------------------------------------------------
void create_stream(const SP_Device* d, SP_Stream* stream, TF_Status* s) {
  if (!use_device(d, s)) return;
  auto* st = new SP_Stream_st{nullptr, d->ordinal};
  if (!hip_ok(hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking), s, "create_stream")) {
    delete st;
    *stream = nullptr;
    return;
  }
  *stream = st;
}

void destroy_stream(const SP_Device* d, SP_Stream stream) {
  if (!stream) return;
  if (use_device(d, nullptr)) (void)hipStreamDestroy(stream->stream);
  delete stream;
}

void create_stream_dependency(const SP_Device* d, SP_Stream dependent, SP_Stream other,
                              TF_Status* s) {
  if (!use_device(d, s)) return;
  if (!dependent || !other) {
    set_error(s, TF_INVALID_ARGUMENT, "create_stream_dependency: null stream");
    return;
  }
  TFMA_Status st;
  if (TFMA_CreateStreamDependency(dependent->stream, other->stream, &st) != TFMA_OK) {
    set_error(s, static_cast<TF_Code>(st.code), "%s", st.message);
    return;
  }
  set_ok(s);
}

void get_stream_status(const SP_Device* d, SP_Stream stream, TF_Status* s) {
  if (!use_device(d, s)) return;
  const hipError_t e = hipStreamQuery(stream->stream);
  if (e == hipSuccess || e == hipErrorNotReady) {
    set_ok(s);
    return;
  }
  set_error(s, TF_INTERNAL, "stream status: %s", hipGetErrorString(e));
}

void create_event(const SP_Device* d, SP_Event* event, TF_Status* s) {
  if (!use_device(d, s)) return;
  auto* ev = new SP_Event_st{nullptr};
  if (!hip_ok(hipEventCreateWithFlags(&ev->event, hipEventDisableTiming), s, "create_event")) {
    delete ev;
    *event = nullptr;
    return;
  }
  *event = ev;
}

void destroy_event(const SP_Device* d, SP_Event event) {
  if (!event) return;
  if (use_device(d, nullptr)) (void)hipEventDestroy(event->event);
  delete event;
}

SE_EventStatus get_event_status(const SP_Device* d, SP_Event event) {
  if (!event || !use_device(d, nullptr)) return SE_EVENT_ERROR;
  const hipError_t e = hipEventQuery(event->event);
  if (e == hipSuccess) return SE_EVENT_COMPLETE;
  if (e == hipErrorNotReady) return SE_EVENT_PENDING;
  return SE_EVENT_ERROR;
}

void record_event(const SP_Device* d, SP_Stream stream, SP_Event event, TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipEventRecord(event->event, stream->stream), s, "record_event");
}

void wait_for_event(const SP_Device* const d, SP_Stream stream, SP_Event event,
                    TF_Status* const s) {
  if (!use_device(d, s)) return;
  hip_ok(hipStreamWaitEvent(stream->stream, event->event, 0), s, "wait_for_event");
}

void block_host_for_event(const SP_Device* d, SP_Event event, TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipEventSynchronize(event->event), s, "block_host_for_event");
}

void block_host_until_done(const SP_Device* d, SP_Stream stream, TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipStreamSynchronize(stream->stream), s, "block_host_until_done");
}

void synchronize_all_activity(const SP_Device* d, TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipDeviceSynchronize(), s, "synchronize_all_activity");
}

// ---------------------------------------------------------------------------
// Timers: a pair of timing events around the interval.
// ---------------------------------------------------------------------------
void create_timer(const SP_Device* d, SP_Timer* timer, TF_Status* s) {
  if (!use_device(d, s)) return;
  auto* t = new SP_Timer_st{nullptr, nullptr};
  if (!hip_ok(hipEventCreate(&t->start), s, "create_timer") ||
      !hip_ok(hipEventCreate(&t->stop), s, "create_timer")) {
    if (t->start) (void)hipEventDestroy(t->start);
    delete t;
    *timer = nullptr;
    return;
  }
  *timer = t;
}

void destroy_timer(const SP_Device* d, SP_Timer timer) {
  if (!timer) return;
  if (use_device(d, nullptr)) {
    (void)hipEventDestroy(timer->start);
    (void)hipEventDestroy(timer->stop);
  }
  delete timer;
}

void start_timer(const SP_Device* d, SP_Stream stream, SP_Timer timer, TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipEventRecord(timer->start, stream->stream), s, "start_timer");
}

void stop_timer(const SP_Device* d, SP_Stream stream, SP_Timer timer, TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipEventRecord(timer->stop, stream->stream), s, "stop_timer");
}

uint64_t timer_nanoseconds(SP_Timer timer) {
  if (!timer || hipEventSynchronize(timer->stop) != hipSuccess) return 0;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, timer->start, timer->stop) != hipSuccess) return 0;
  return static_cast<uint64_t>(static_cast<double>(ms) * 1e6);
}

void create_timer_fns(const SP_Platform*, SP_TimerFns* t, TF_Status* s) {
  if (!t) {
    set_error(s, TF_INVALID_ARGUMENT, "create_timer_fns: null timer fns");
    return;
  }
  t->struct_size = SP_TIMER_FNS_STRUCT_SIZE;
  t->nanoseconds = timer_nanoseconds;
  set_ok(s);
}

void destroy_timer_fns(const SP_Platform*, SP_TimerFns*) {}

// ---------------------------------------------------------------------------
// Copies and fills.  Host <-> device copies go through the library's staged
// host path (pageable sources are staged through pinned blocks, so the call
// returns once the source may be reused).
// ---------------------------------------------------------------------------
void copy_status(const TFMA_Status& st, TF_Status* s) {
  if (st.code == TFMA_OK)
    set_ok(s);
  else
    set_error(s, static_cast<TF_Code>(st.code), "%s", st.message);
}

void memcpy_dtoh(const SP_Device* d, SP_Stream stream, void* host_dst,
                 const SP_DeviceMemoryBase* src, uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  TFMA_Status st;
  TFMA_MemcpyDtoH(stream->stream, host_dst, src->opaque, size, 0, &st);
  copy_status(st, s);
}

void memcpy_htod(const SP_Device* d, SP_Stream stream, SP_DeviceMemoryBase* dst,
                 const void* host_src, uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  TFMA_Status st;
  TFMA_MemcpyHtoD(stream->stream, dst->opaque, host_src, size, 0, &st);
  copy_status(st, s);
}

void memcpy_dtod(const SP_Device* d, SP_Stream stream, SP_DeviceMemoryBase* dst,
                 const SP_DeviceMemoryBase* src, uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  if (size == 0) {
    set_ok(s);
    return;
  }
  hip_ok(hipMemcpyAsync(dst->opaque, src->opaque, size, hipMemcpyDeviceToDevice, stream->stream),
         s, "memcpy_dtod");
}

void sync_memcpy_dtoh(const SP_Device* d, void* host_dst, const SP_DeviceMemoryBase* src,
                      uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  TFMA_Status st;
  TFMA_MemcpyDtoH(nullptr, host_dst, src->opaque, size, 1, &st);
  copy_status(st, s);
}

void sync_memcpy_htod(const SP_Device* d, SP_DeviceMemoryBase* dst, const void* host_src,
                      uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  TFMA_Status st;
  TFMA_MemcpyHtoD(nullptr, dst->opaque, host_src, size, 1, &st);
  copy_status(st, s);
}

void sync_memcpy_dtod(const SP_Device* d, SP_DeviceMemoryBase* dst,
                      const SP_DeviceMemoryBase* src, uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  if (size == 0) {
    set_ok(s);
    return;
  }
  hip_ok(hipMemcpy(dst->opaque, src->opaque, size, hipMemcpyDeviceToDevice), s,
         "sync_memcpy_dtod");
}

void mem_zero(const SP_Device* d, SP_Stream stream, SP_DeviceMemoryBase* loc, uint64_t size,
              TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipMemsetAsync(loc->opaque, 0, size, stream->stream), s, "mem_zero");
}

void memset8(const SP_Device* d, SP_Stream stream, SP_DeviceMemoryBase* loc, uint8_t pattern,
             uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  hip_ok(hipMemsetAsync(loc->opaque, pattern, size, stream->stream), s, "memset");
}

void memset32(const SP_Device* d, SP_Stream stream, SP_DeviceMemoryBase* loc, uint32_t pattern,
              uint64_t size, TF_Status* s) {
  if (!use_device(d, s)) return;
  if (size % 4 != 0) {
    set_error(s, TF_INVALID_ARGUMENT, "memset32: size %llu is not a multiple of 4",
              static_cast<unsigned long long>(size));
    return;
  }
  hip_ok(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(loc->opaque),
                           static_cast<int>(pattern), size / 4, stream->stream),
         s, "memset32");
}

// TensorFlow's callback takes a TF_Status it owns for the call.
struct HostCall {
  SE_StatusCallbackFn fn;
  void* arg;
};

void run_host_call(void* p) {
  auto* hc = static_cast<HostCall*>(p);
  TF_Status* st = TF_NewStatus();
  hc->fn(hc->arg, st);
  TF_DeleteStatus(st);
  delete hc;
}

TF_Bool host_callback(const SP_Device* d, SP_Stream stream, SE_StatusCallbackFn fn, void* arg) {
  if (!fn || !stream || !use_device(d, nullptr)) return 0;
  auto* hc = new HostCall{fn, arg};
  TFMA_Status st;
  if (TFMA_HostCallback(stream->stream, run_host_call, hc, &st) != TFMA_OK) {
    delete hc;
    return 0;
  }
  return 1;
}

void create_stream_executor(const SP_Platform*, SE_CreateStreamExecutorParams* p, TF_Status* s) {
  if (!p || !p->stream_executor) {
    set_error(s, TF_INVALID_ARGUMENT, "create_stream_executor: null params");
    return;
  }
  if (p->struct_size < SE_CREATE_STREAM_EXECUTOR_PARAMS_STRUCT_SIZE ||
      p->stream_executor->struct_size < SP_STREAMEXECUTOR_STRUCT_SIZE) {
    set_error(s, TF_INVALID_ARGUMENT, "create_stream_executor: struct_size too small");
    return;
  }
  SP_StreamExecutor* se = p->stream_executor;
  se->struct_size = SP_STREAMEXECUTOR_STRUCT_SIZE;
  se->allocate = allocate;
  se->deallocate = deallocate;
  se->host_memory_allocate = host_memory_allocate;
  se->host_memory_deallocate = host_memory_deallocate;
  se->unified_memory_allocate = unified_memory_allocate;
  se->unified_memory_deallocate = unified_memory_deallocate;
  se->get_allocator_stats = get_allocator_stats;
  se->device_memory_usage = device_memory_usage;
  se->create_stream = create_stream;
  se->destroy_stream = destroy_stream;
  se->create_stream_dependency = create_stream_dependency;
  se->get_stream_status = get_stream_status;
  se->create_event = create_event;
  se->destroy_event = destroy_event;
  se->get_event_status = get_event_status;
  se->record_event = record_event;
  se->wait_for_event = wait_for_event;
  se->create_timer = create_timer;
  se->destroy_timer = destroy_timer;
  se->start_timer = start_timer;
  se->stop_timer = stop_timer;
  se->memcpy_dtoh = memcpy_dtoh;
  se->memcpy_htod = memcpy_htod;
  se->memcpy_dtod = memcpy_dtod;
  se->sync_memcpy_dtoh = sync_memcpy_dtoh;
  se->sync_memcpy_htod = sync_memcpy_htod;
  se->sync_memcpy_dtod = sync_memcpy_dtod;
  se->block_host_for_event = block_host_for_event;
  se->block_host_until_done = block_host_until_done;
  se->synchronize_all_activity = synchronize_all_activity;
  se->mem_zero = mem_zero;
  se->memset = memset8;
  se->memset32 = memset32;
  se->host_callback = host_callback;
  set_ok(s);
}

void destroy_stream_executor(const SP_Platform*, SP_StreamExecutor*) {}
void destroy_platform(SP_Platform*) {}
void destroy_platform_fns(SP_PlatformFns*) {}

}  // namespace

// ===========================================================================
// Kernels.
// ===========================================================================
namespace {

// A TF_Tensor* owned for the duration of a compute call.
class Tensor {
 public:
  Tensor() = default;
  explicit Tensor(TF_Tensor* t) : t_(t) {}
  Tensor(const Tensor&) = delete;
  Tensor& operator=(const Tensor&) = delete;
  Tensor(Tensor&& o) noexcept : t_(o.t_) { o.t_ = nullptr; }
  Tensor& operator=(Tensor&& o) noexcept {
    reset(o.t_);
    o.t_ = nullptr;
    return *this;
  }
  ~Tensor() { reset(nullptr); }
  void reset(TF_Tensor* t) {
    if (t_) TF_DeleteTensor(t_);
    t_ = t;
  }
  TF_Tensor* get() const { return t_; }
  TF_Tensor** out() {
    reset(nullptr);
    return &t_;
  }
  explicit operator bool() const { return t_ != nullptr; }
  int ndims() const { return TF_NumDims(t_); }
  int64_t dim(int i) const { return TF_Dim(t_, i); }
  int64_t elements() const { return TF_TensorElementCount(t_); }
  TF_DataType dtype() const { return TF_TensorType(t_); }
  void* data() const { return TF_TensorData(t_); }
  std::vector<int64_t> shape() const {
    std::vector<int64_t> s(ndims());
    for (int i = 0; i < ndims(); ++i) s[i] = dim(i);
    return s;
  }
  // The C ABI's descriptor (rank <= TFMA_MAX_DIMS, checked by the caller).
  TFMA_Tensor desc() const {
    TFMA_Tensor d{};
    d.data = t_ ? data() : nullptr;
    d.dtype = t_ ? static_cast<int32_t>(dtype()) : 0;
    d.ndims = t_ ? ndims() : 0;
    for (int i = 0; i < d.ndims && i < TFMA_MAX_DIMS; ++i) d.dims[i] = dim(i);
    return d;
  }

 private:
  TF_Tensor* t_ = nullptr;
};

// Per-call context: the kernel context, one TF_Status, the stream.
class Call {
 public:
  explicit Call(TF_OpKernelContext* ctx) : ctx_(ctx), st_(TF_NewStatus()) {}
  ~Call() { TF_DeleteStatus(st_); }
  TF_OpKernelContext* ctx() const { return ctx_; }
  TF_Status* status() const { return st_; }

  // Reports the current status to TensorFlow if it is not OK.
  bool check() {
    if (TF_GetCode(st_) == TF_OK) return true;
    TF_OpKernelContext_Failure(ctx_, st_);
    return false;
  }
  bool fail(TF_Code code, const char* msg) {
    TF_SetStatus(st_, code, msg);
    TF_OpKernelContext_Failure(ctx_, st_);
    return false;
  }
  bool check(int code, const TFMA_Status& s) {
    if (code == TFMA_OK) return true;
    return fail(static_cast<TF_Code>(code), s.message);
  }
  // Reports the library's validation error for arguments the adapter has
  // found invalid (the call gets a null stream and is expected to fail
  // before any launch; if it does not, `fallback` is reported).
  template <class Fn>
  void reject(Fn&& fn, const char* fallback) {
    TFMA_Status st;
    const int rc = fn(&st);
    if (rc != TFMA_OK)
      fail(static_cast<TF_Code>(rc), st.message);
    else
      fail(TF_INVALID_ARGUMENT, fallback);
  }

  // The op's stream, with its device made current.
  bool stream(hipStream_t* out) {
    SP_Stream s = TF_GetStream(ctx_, st_);
    if (!check()) return false;
    if (!s) return fail(TF_INTERNAL, "no stream for the kernel");
    if (hipSetDevice(s->device) != hipSuccess) return fail(TF_INTERNAL, "hipSetDevice failed");
    *out = s->stream;
    return true;
  }

  bool input(int i, Tensor* t) {
    TF_GetInput(ctx_, i, t->out(), st_);
    return check();
  }

  bool ranks_ok(std::initializer_list<const Tensor*> ts) {
    for (const Tensor* t : ts)
      if (t->ndims() > TFMA_MAX_DIMS) return fail(TF_UNIMPLEMENTED, "rank above 8");
    return true;
  }

  bool output(int i, TF_DataType dt, const std::vector<int64_t>& shape, Tensor* t) {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    const size_t es = dt == TF_UINT8 ? 1
                      : dt == TF_HALF || dt == TF_BFLOAT16 ? 2
                      : dt == TF_DOUBLE || dt == TF_INT64  ? 8
                                                           : 4;
    t->reset(TF_AllocateOutput(ctx_, i, dt, shape.data(), static_cast<int>(shape.size()),
                               static_cast<size_t>(n) * es, st_));
    return check();
  }

  // Output i aliasing one of `candidates` when TensorFlow allows it (the
  // elementwise kernels read element i before writing element i).
  bool forward_or_output(std::initializer_list<int> candidates, int i,
                         const std::vector<int64_t>& shape, Tensor* t) {
    std::vector<int> c(candidates);
    int fwd = -1;
    t->reset(TF_ForwardInputOrAllocateOutput(ctx_, c.data(), static_cast<int>(c.size()), i,
                                             shape.data(), static_cast<int>(shape.size()),
                                             &fwd, st_));
    return check();
  }

  // Device scratch of `bytes` (TensorFlow's allocate_temp).
  bool temp(size_t bytes, Tensor* t) {
    const int64_t dims[1] = {static_cast<int64_t>(bytes > 0 ? bytes : 1)};
    TF_AllocatorAttributes attrs{TF_ALLOCATOR_ATTRIBUTES_STRUCT_SIZE, 0};
    t->reset(TF_AllocateTemp(ctx_, TF_UINT8, dims, 1, &attrs, st_));
    return check();
  }

 private:
  TF_OpKernelContext* ctx_;
  TF_Status* st_;
};

// Attribute reads at kernel construction.
struct Attrs {
  TF_OpKernelConstruction* c;
  TF_Status* st;
  bool ok = true;
  explicit Attrs(TF_OpKernelConstruction* ctx) : c(ctx), st(TF_NewStatus()) {}
  ~Attrs() {
    if (!ok) TF_OpKernelConstruction_Failure(c, st);
    TF_DeleteStatus(st);
  }
  bool has(const char* name) {
    TF_Status* s = TF_NewStatus();
    const bool h = TF_OpKernelConstruction_HasAttr(c, name, s) != 0;
    TF_DeleteStatus(s);
    return h;
  }
  float f(const char* name, float dflt) {
    if (!ok || !has(name)) return dflt;
    float v = dflt;
    TF_OpKernelConstruction_GetAttrFloat(c, name, &v, st);
    ok = TF_GetCode(st) == TF_OK;
    return v;
  }
  bool b(const char* name, bool dflt) {
    if (!ok || !has(name)) return dflt;
    TF_Bool v = dflt ? 1 : 0;
    TF_OpKernelConstruction_GetAttrBool(c, name, &v, st);
    ok = TF_GetCode(st) == TF_OK;
    return v != 0;
  }
  int32_t i32(const char* name, int32_t dflt) {
    if (!ok || !has(name)) return dflt;
    int32_t v = dflt;
    TF_OpKernelConstruction_GetAttrInt32(c, name, &v, st);
    ok = TF_GetCode(st) == TF_OK;
    return v;
  }
  std::string str(const char* name, const char* dflt) {
    if (!ok || !has(name)) return dflt;
    char buf[64] = {0};
    TF_OpKernelConstruction_GetAttrString(c, name, buf, sizeof(buf) - 1, st);
    ok = TF_GetCode(st) == TF_OK;
    return buf;
  }
};

template <class K>
void delete_kernel(void* k) {
  delete static_cast<K*>(k);
}

// ---- FusedBatchNorm / V2 / V3 ---------------------------------------------
struct BnKernel {
  float epsilon = 1e-4f;
  float exponential_avg_factor = 1.0f;
  std::string data_format = "NHWC";
  bool is_training = true;
  bool v3 = false;  // outputs reserve_space_3 (forward) / takes it (grad)
};

template <bool kV3>
void* bn_create(TF_OpKernelConstruction* c) {
  auto* k = new BnKernel();
  Attrs a(c);
  k->epsilon = a.f("epsilon", 1e-4f);
  k->exponential_avg_factor = a.f("exponential_avg_factor", 1.0f);
  k->data_format = a.str("data_format", "NHWC");
  k->is_training = a.b("is_training", true);
  k->v3 = kV3;
  return k;
}

int64_t channels_of(const Tensor& x, const std::string& fmt) {
  if (x.ndims() < 2) return 0;
  return (fmt == "NCHW" || fmt == "NCDHW") ? x.dim(1) : x.dim(x.ndims() - 1);
}

void bn_forward_compute(void* kernel, TF_OpKernelContext* ctx) {
  const BnKernel& k = *static_cast<BnKernel*>(kernel);
  Call call(ctx);
  Tensor x, scale, offset, mean, var;
  if (!call.input(0, &x) || !call.input(1, &scale) || !call.input(2, &offset) ||
      !call.input(3, &mean) || !call.input(4, &var))
    return;
  if (!call.ranks_ok({&x}) || x.ndims() < 2) {
    call.fail(TF_INVALID_ARGUMENT, "input must be 4 or 5-dimensional");
    return;
  }
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  const int64_t c = channels_of(x, k.data_format);
  Tensor y, bm, bv, r1, r2, r3;
  if (!call.output(0, x.dtype(), x.shape(), &y) || !call.output(1, TF_FLOAT, {c}, &bm) ||
      !call.output(2, TF_FLOAT, {c}, &bv) || !call.output(3, TF_FLOAT, {c}, &r1) ||
      !call.output(4, TF_FLOAT, {c}, &r2))
    return;
  if (k.v3 && !call.output(5, TF_FLOAT, {}, &r3)) return;
  TFMA_Tensor dx = x.desc(), ds = scale.desc(), doff = offset.desc(), dm = mean.desc(),
              dv = var.desc(), dy = y.desc(), dbm = bm.desc(), dbv = bv.desc(), d1 = r1.desc(),
              d2 = r2.desc(), d3 = r3.desc();
  TFMA_Status st;
  size_t ws_bytes = 0;
  if (!call.check(TFMA_FusedBatchNormWorkspaceBytes(&dx, k.data_format.c_str(), &ws_bytes, &st),
                  st))
    return;
  Tensor ws;
  if (!call.temp(ws_bytes, &ws)) return;
  const int rc = TFMA_FusedBatchNormV3(stream, &dx, &ds, &doff, &dm, &dv, k.epsilon,
                                       k.exponential_avg_factor, k.data_format.c_str(),
                                       k.is_training ? 1 : 0, &dy, &dbm, &dbv, &d1, &d2,
                                       k.v3 ? &d3 : nullptr, ws.data(), ws_bytes, &st);
  call.check(rc, st);
}

void bn_grad_compute(void* kernel, TF_OpKernelContext* ctx) {
  const BnKernel& k = *static_cast<BnKernel*>(kernel);
  Call call(ctx);
  Tensor dy, x, scale, r1, r2, r3;
  if (!call.input(0, &dy) || !call.input(1, &x) || !call.input(2, &scale) ||
      !call.input(3, &r1) || !call.input(4, &r2))
    return;
  if (k.v3 && !call.input(5, &r3)) return;
  if (!call.ranks_ok({&x, &dy}) || x.ndims() < 2) {
    call.fail(TF_INVALID_ARGUMENT, "input must be 4 or 5-dimensional");
    return;
  }
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  const int64_t c = channels_of(x, k.data_format);
  Tensor dx, dscale, doffset, r4, r5;
  // reserve_space_4/5 are the empty placeholders TensorFlow's kernels emit.
  if (!call.output(0, x.dtype(), x.shape(), &dx) || !call.output(1, TF_FLOAT, {c}, &dscale) ||
      !call.output(2, TF_FLOAT, {c}, &doffset) || !call.output(3, TF_FLOAT, {0}, &r4) ||
      !call.output(4, TF_FLOAT, {0}, &r5))
    return;
  TFMA_Tensor ddy = dy.desc(), dxin = x.desc(), ds = scale.desc(), d1 = r1.desc(),
              d2 = r2.desc(), d3 = r3.desc(), ddx = dx.desc(), dsc = dscale.desc(),
              dof = doffset.desc(), d4 = r4.desc(), d5 = r5.desc();
  TFMA_Status st;
  size_t ws_bytes = 0;
  if (!call.check(
          TFMA_FusedBatchNormWorkspaceBytes(&dxin, k.data_format.c_str(), &ws_bytes, &st), st))
    return;
  Tensor ws;
  if (!call.temp(ws_bytes, &ws)) return;
  const int rc = TFMA_FusedBatchNormGradV3(
      stream, &ddy, &dxin, &ds, &d1, &d2, k.v3 ? &d3 : nullptr, k.epsilon,
      k.data_format.c_str(), k.is_training ? 1 : 0, &ddx, &dsc, &dof, &d4, &d5, ws.data(),
      ws_bytes, &st);
  call.check(rc, st);
}

// ---- Adam -----------------------------------------------------------------
struct AdamKernel {
  bool use_locking = false;
  bool use_nesterov = false;
  int n = 1;  // tensors per kind (grouped op)
};

void* adam_create(TF_OpKernelConstruction* c) {
  auto* k = new AdamKernel();
  Attrs a(c);
  k->use_locking = a.b("use_locking", false);
  k->use_nesterov = a.b("use_nesterov", false);
  k->n = a.i32("N", 1);
  return k;
}

// Copy-on-read hook TensorFlow calls when a variable's buffer is shared and
// must be copied before the in-place update.
void copy_variable(TF_OpKernelContext* ctx, TF_Tensor* source, TF_Tensor* dest) {
  TF_Status* s = TF_NewStatus();
  SP_Stream sp = TF_GetStream(ctx, s);
  if (TF_GetCode(s) == TF_OK && sp) {
    (void)hipSetDevice(sp->device);
    (void)hipMemcpyAsync(TF_TensorData(dest), TF_TensorData(source), TF_TensorByteSize(source),
                         hipMemcpyDeviceToDevice, sp->stream);
  }
  TF_DeleteStatus(s);
}

// The variables' locks, held for the whole update when use_locking (taken
// by TensorFlow in a fixed order, as MaybeLockVariableInputMutexesInOrder).
class VariableLocks {
 public:
  ~VariableLocks() {
    if (h_) TF_ReleaseVariableInputLockHolder(h_);
  }
  bool lock(Call& call, std::vector<int> inputs) {
    TF_MaybeLockVariableInput(call.ctx(), inputs.data(), inputs.size(), false, false,
                              copy_variable, &h_, call.status());
    return call.check();
  }

 private:
  TF_VariableInputLockHolder* h_ = nullptr;
};

bool variable(Call& call, int input, bool locked, Tensor* t) {
  TF_GetInputTensorFromVariable(call.ctx(), input, locked, false, false, copy_variable, t->out(),
                                call.status());
  return call.check();
}

// ResourceApplyAdam, ApplyAdam (reference variables) and
// MusaResourceApplyAdamMixed: var 0, m 1, v 2, beta1_power .. epsilon 3-8
// (host memory), grad 9.
template <bool kMixed>
void adam_compute(void* kernel, TF_OpKernelContext* ctx) {
  const AdamKernel& k = *static_cast<AdamKernel*>(kernel);
  Call call(ctx);
  VariableLocks locks;
  if (k.use_locking && !locks.lock(call, {0, 1, 2})) return;
  Tensor var, m, v, grad, sc[6];
  if (!variable(call, 0, k.use_locking, &var) || !variable(call, 1, k.use_locking, &m) ||
      !variable(call, 2, k.use_locking, &v))
    return;
  for (int i = 0; i < 6; ++i)
    if (!call.input(3 + i, &sc[i])) return;
  if (!call.input(9, &grad)) return;
  if (!call.ranks_ok({&var, &m, &v, &grad})) return;
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  TFMA_Tensor dvar = var.desc(), dm = m.desc(), dv = v.desc(), dg = grad.desc(), ds[6];
  for (int i = 0; i < 6; ++i) ds[i] = sc[i].desc();
  TFMA_Status st;
  // TensorFlow's variable locks are held when use_locking: the library's
  // own striped locks are not needed on top.
  const int rc =
      kMixed ? TFMA_MusaResourceApplyAdamMixed(stream, &dvar, &dm, &dv, &ds[0], &ds[1], &ds[2],
                                               &ds[3], &ds[4], &ds[5], &dg, 0,
                                               k.use_nesterov ? 1 : 0, &st)
             : TFMA_ResourceApplyAdam(stream, &dvar, &dm, &dv, &ds[0], &ds[1], &ds[2], &ds[3],
                                      &ds[4], &ds[5], &dg, 0, k.use_nesterov ? 1 : 0, &st);
  call.check(rc, st);
}

// MusaGroupedResourceApplyAdam: vars [0, N), ms [N, 2N), vs [2N, 3N),
// beta1_power .. epsilon [3N, 3N+6) (host memory), grads [3N+6, 4N+6).
void grouped_adam_compute(void* kernel, TF_OpKernelContext* ctx) {
  const AdamKernel& k = *static_cast<AdamKernel*>(kernel);
  const int n = k.n;
  Call call(ctx);
  if (n < 1) {
    call.fail(TF_INVALID_ARGUMENT, "N must be >= 1");
    return;
  }
  VariableLocks locks;
  if (k.use_locking) {
    std::vector<int> ids(3 * n);
    for (int i = 0; i < 3 * n; ++i) ids[i] = i;
    if (!locks.lock(call, ids)) return;
  }
  std::vector<Tensor> state(3 * n), grads(n);
  Tensor sc[6];
  for (int i = 0; i < 3 * n; ++i)
    if (!variable(call, i, k.use_locking, &state[i])) return;
  for (int i = 0; i < 6; ++i)
    if (!call.input(3 * n + i, &sc[i])) return;
  for (int i = 0; i < n; ++i)
    if (!call.input(3 * n + 6 + i, &grads[i])) return;
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  std::vector<TFMA_Tensor> dvars(n), dms(n), dvs(n), dgs(n);
  for (int i = 0; i < n; ++i) {
    if (!call.ranks_ok({&state[i], &state[n + i], &state[2 * n + i], &grads[i]})) return;
    dvars[i] = state[i].desc();
    dms[i] = state[n + i].desc();
    dvs[i] = state[2 * n + i].desc();
    dgs[i] = grads[i].desc();
  }
  TFMA_Tensor ds[6];
  for (int i = 0; i < 6; ++i) ds[i] = sc[i].desc();
  TFMA_Status st;
  size_t ws_bytes = 0;
  if (!call.check(TFMA_GroupedApplyAdamWorkspaceBytes(n, dvars.data(), &ws_bytes, &st), st))
    return;
  Tensor ws;
  if (!call.temp(ws_bytes, &ws)) return;
  const int rc = TFMA_GroupedResourceApplyAdam(
      stream, n, dvars.data(), dms.data(), dvs.data(), dgs.data(), &ds[0], &ds[1], &ds[2], &ds[3],
      &ds[4], &ds[5], 0, k.use_nesterov ? 1 : 0, ws.data(), ws_bytes, &st);
  call.check(rc, st);
}

// ---- Elementwise ----------------------------------------------------------
struct FormatKernel {
  std::string data_format = "NHWC";
};

void* format_create(TF_OpKernelConstruction* c) {
  auto* k = new FormatKernel();
  Attrs a(c);
  k->data_format = a.str("data_format", "NHWC");
  return k;
}

void* plain_create(TF_OpKernelConstruction*) { return new FormatKernel(); }

// Broadcast shape of the inputs (right-aligned, TensorFlow's BCast rule);
// false if they do not broadcast.
bool broadcast(const std::vector<const Tensor*>& ins, std::vector<int64_t>* out) {
  size_t rank = 0;
  for (const Tensor* t : ins) rank = std::max(rank, static_cast<size_t>(t->ndims()));
  out->assign(rank, 1);
  for (const Tensor* t : ins) {
    const int nd = t->ndims();
    for (int i = 0; i < nd; ++i) {
      int64_t& o = (*out)[rank - nd + i];
      const int64_t d = t->dim(i);
      if (d == o || d == 1) continue;
      if (o == 1) {
        o = d;
        continue;
      }
      return false;
    }
  }
  return true;
}

using BinaryFn = int (*)(void*, const TFMA_Tensor*, const TFMA_Tensor*, TFMA_Tensor*,
                         TFMA_Status*);

template <BinaryFn kFn>
void binary_compute(void*, TF_OpKernelContext* ctx) {
  Call call(ctx);
  Tensor a, b;
  if (!call.input(0, &a) || !call.input(1, &b) || !call.ranks_ok({&a, &b})) return;
  std::vector<int64_t> shape;
  if (!broadcast({&a, &b}, &shape)) {
    TFMA_Tensor da = a.desc(), db = b.desc(), dz = da;
    dz.data = nullptr;
    call.reject([&](TFMA_Status* st) { return kFn(nullptr, &da, &db, &dz, st); },
                "Incompatible shapes");
    return;
  }
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  Tensor z;
  std::vector<int> cand;
  if (a.shape() == shape) cand.push_back(0);
  if (b.shape() == shape) cand.push_back(1);
  bool ok;
  if (cand.size() == 2)
    ok = call.forward_or_output({0, 1}, 0, shape, &z);
  else if (cand.size() == 1)
    ok = call.forward_or_output({cand[0]}, 0, shape, &z);
  else
    ok = call.output(0, a.dtype(), shape, &z);
  if (!ok) return;
  TFMA_Tensor da = a.desc(), db = b.desc(), dz = z.desc();
  TFMA_Status st;
  call.check(kFn(stream, &da, &db, &dz, &st), st);
}

void relu_compute(void*, TF_OpKernelContext* ctx) {
  Call call(ctx);
  Tensor x;
  if (!call.input(0, &x) || !call.ranks_ok({&x})) return;
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  Tensor y;
  if (!call.forward_or_output({0}, 0, x.shape(), &y)) return;
  TFMA_Tensor dx = x.desc(), dy = y.desc();
  TFMA_Status st;
  call.check(TFMA_Relu(stream, &dx, &dy, &st), st);
}

template <bool kRelu>
void bias_add_compute(void* kernel, TF_OpKernelContext* ctx) {
  const FormatKernel& k = *static_cast<FormatKernel*>(kernel);
  Call call(ctx);
  Tensor value, bias;
  if (!call.input(0, &value) || !call.input(1, &bias) || !call.ranks_ok({&value, &bias})) return;
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  Tensor out;
  if (!call.forward_or_output({0}, 0, value.shape(), &out)) return;
  TFMA_Tensor dv = value.desc(), db = bias.desc(), dout = out.desc();
  TFMA_Status st;
  const int rc = kRelu ? TFMA_MusaBiasAddRelu(stream, &dv, &db, k.data_format.c_str(), &dout, &st)
                       : TFMA_BiasAdd(stream, &dv, &db, k.data_format.c_str(), &dout, &st);
  call.check(rc, st);
}

void shifted_affine_map_compute(void*, TF_OpKernelContext* ctx) {
  Call call(ctx);
  Tensor a, b, c;
  if (!call.input(0, &a) || !call.input(1, &b) || !call.input(2, &c) ||
      !call.ranks_ok({&a, &b, &c}))
    return;
  std::vector<int64_t> shape;
  TFMA_Tensor da = a.desc(), db = b.desc(), dc = c.desc();
  if (!broadcast({&a, &b, &c}, &shape)) {
    TFMA_Tensor dout = da;
    dout.data = nullptr;
    call.reject(
        [&](TFMA_Status* st) { return TFMA_MusaShiftedAffineMap(nullptr, &da, &db, &dc, &dout, st); },
        "Incompatible shapes");
    return;
  }
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  Tensor out;
  if (!call.output(0, a.dtype(), shape, &out)) return;
  TFMA_Tensor dout = out.desc();
  TFMA_Status st;
  call.check(TFMA_MusaShiftedAffineMap(stream, &da, &db, &dc, &dout, &st), st);
}

void relu_grad_compute(void*, TF_OpKernelContext* ctx) {
  Call call(ctx);
  Tensor g, f;
  if (!call.input(0, &g) || !call.input(1, &f) || !call.ranks_ok({&g, &f})) return;
  TFMA_Tensor dg = g.desc(), df = f.desc();
  if (g.shape() != f.shape()) {
    TFMA_Tensor dout = dg;
    dout.data = nullptr;
    call.reject([&](TFMA_Status* st) { return TFMA_ReluGrad(nullptr, &dg, &df, &dout, st); },
                "Inputs to ReluGrad must have the same shape");
    return;
  }
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  Tensor out;
  if (!call.forward_or_output({0}, 0, g.shape(), &out)) return;
  TFMA_Tensor dout = out.desc();
  TFMA_Status st;
  call.check(TFMA_ReluGrad(stream, &dg, &df, &dout, &st), st);
}

void bias_add_grad_compute(void* kernel, TF_OpKernelContext* ctx) {
  const FormatKernel& k = *static_cast<FormatKernel*>(kernel);
  Call call(ctx);
  Tensor x;
  if (!call.input(0, &x) || !call.ranks_ok({&x})) return;
  TFMA_Tensor dx = x.desc();
  TFMA_Status st;
  size_t ws_bytes = 0;
  if (!call.check(TFMA_BiasAddGradWorkspaceBytes(&dx, k.data_format.c_str(), &ws_bytes, &st),
                  st))
    return;
  hipStream_t stream;
  if (!call.stream(&stream)) return;
  const int cd = (k.data_format == "NCHW" && x.ndims() > 1) ? 1 : x.ndims() - 1;
  Tensor out, ws;
  if (!call.output(0, x.dtype(), {x.dim(cd)}, &out) || !call.temp(ws_bytes, &ws)) return;
  TFMA_Tensor dout = out.desc();
  call.check(TFMA_BiasAddGrad(stream, &dx, k.data_format.c_str(), &dout, ws.data(), ws_bytes,
                              &st),
             st);
}

// ---- Registration ---------------------------------------------------------
struct KernelSpec {
  const char* op;
  void* (*create)(TF_OpKernelConstruction*);
  void (*compute)(void*, TF_OpKernelContext*);
  void (*destroy)(void*);
  std::vector<std::pair<const char*, TF_DataType>> types;
  std::vector<const char*> host_memory;
};

bool register_kernel(const KernelSpec& k, TF_Status* s) {
  TF_KernelBuilder* b = TF_NewKernelBuilder(k.op, kDeviceType, k.create, k.compute, k.destroy);
  for (const auto& t : k.types) {
    TF_KernelBuilder_TypeConstraint(b, t.first, t.second, s);
    if (TF_GetCode(s) != TF_OK) {
      TF_DeleteKernelBuilder(b);
      return false;
    }
  }
  for (const char* h : k.host_memory) TF_KernelBuilder_HostMemory(b, h);
  // The builder belongs to TensorFlow once registered.
  TF_RegisterKernelBuilder(k.op, b, s);
  return TF_GetCode(s) == TF_OK;
}

// Output 0 has input 0's shape.
void same_shape_fn(TF_ShapeInferenceContext* ctx, TF_Status* s) {
  TF_ShapeHandle* h = TF_NewShapeHandle();
  TF_ShapeInferenceContextGetInput(ctx, 0, h, s);
  if (TF_GetCode(s) == TF_OK) TF_ShapeInferenceContextSetOutput(ctx, 0, h, s);
  TF_DeleteShapeHandle(h);
}

// Output 0: the input every other input broadcasts to, if there is one with
// all dimensions known; otherwise an unknown shape (the kernel computes the
// broadcast shape at run time).
void broadcast_shape_fn(TF_ShapeInferenceContext* ctx, TF_Status* s) {
  const int n = static_cast<int>(TF_ShapeInferenceContextNumInputs(ctx));
  std::vector<TF_ShapeHandle*> hs(n);
  std::vector<std::vector<int64_t>> dims(n);
  bool known = true;
  for (int i = 0; i < n; ++i) {
    hs[i] = TF_NewShapeHandle();
    TF_ShapeInferenceContextGetInput(ctx, i, hs[i], s);
    if (TF_GetCode(s) != TF_OK || !TF_ShapeInferenceContextRankKnown(ctx, hs[i])) {
      known = false;
      continue;
    }
    const int64_t r = TF_ShapeInferenceContextRank(ctx, hs[i]);
    TF_DimensionHandle* d = TF_NewDimensionHandle();
    for (int64_t j = 0; j < r; ++j) {
      TF_ShapeInferenceContextDim(ctx, hs[i], j, d);
      if (!TF_DimensionHandleValueKnown(d)) known = false;
      dims[i].push_back(TF_DimensionHandleValue(d));
    }
    TF_DeleteDimensionHandle(d);
  }
  int pick = -1;
  if (known && TF_GetCode(s) == TF_OK) {
    for (int i = 0; i < n && pick < 0; ++i) {
      bool all = true;
      for (int j = 0; j < n && all; ++j) {
        if (dims[j].size() > dims[i].size()) {
          all = false;
          break;
        }
        const size_t off = dims[i].size() - dims[j].size();
        for (size_t q = 0; q < dims[j].size(); ++q)
          if (dims[j][q] != 1 && dims[j][q] != dims[i][off + q]) all = false;
      }
      if (all) pick = i;
    }
  }
  if (TF_GetCode(s) == TF_OK) {
    if (pick >= 0)
      TF_ShapeInferenceContextSetOutput(ctx, 0, hs[pick], s);
    else
      TF_ShapeInferenceContextSetUnknownShape(ctx, s);
  }
  for (TF_ShapeHandle* h : hs) TF_DeleteShapeHandle(h);
}

void no_output_shape_fn(TF_ShapeInferenceContext*, TF_Status* s) { TF_SetStatus(s, TF_OK, ""); }

struct OpSpec {
  const char* name;
  std::vector<const char*> inputs, outputs, attrs;
  void (*shape_fn)(TF_ShapeInferenceContext*, TF_Status*);
  bool stateful;
};

// Op definitions of the ops TensorFlow does not have.  An op that is already
// defined (for example by another plugin that registers the reference's
// ops) is left as it is.
bool register_op(const OpSpec& o, TF_Status* s) {
  TF_OpDefinitionBuilder* b = TF_NewOpDefinitionBuilder(o.name);
  for (const char* i : o.inputs) TF_OpDefinitionBuilderAddInput(b, i);
  for (const char* i : o.outputs) TF_OpDefinitionBuilderAddOutput(b, i);
  for (const char* a : o.attrs) TF_OpDefinitionBuilderAddAttr(b, a);
  if (o.stateful) TF_OpDefinitionBuilderSetIsStateful(b, true);
  TF_OpDefinitionBuilderSetShapeInferenceFunction(b, o.shape_fn);
  TF_RegisterOpDefinition(b, s);
  if (TF_GetCode(s) == TF_ALREADY_EXISTS) TF_SetStatus(s, TF_OK, "");
  return TF_GetCode(s) == TF_OK;
}

const std::vector<OpSpec>& op_specs() {
  static const std::vector<OpSpec> specs = {
      {"MusaBiasAddRelu",
       {"value: T", "bias: T"},
       {"output: T"},
       {"T: {float, half, bfloat16, double}", "data_format: {'NHWC', 'NCHW'} = 'NHWC'"},
       same_shape_fn,
       false},
      {"MusaAddV2Relu",
       {"x: T", "y: T"},
       {"z: T"},
       {"T: {float, half, bfloat16, double}"},
       broadcast_shape_fn,
       false},
      {"MusaShiftedAffineMap",
       {"data_left: T", "mask: T", "sliced_var_right: T"},
       {"output: T"},
       {"T: {float, double, half, bfloat16}"},
       broadcast_shape_fn,
       false},
      {"MusaResourceApplyAdamMixed",
       {"var: resource", "m: resource", "v: resource", "beta1_power: float",
        "beta2_power: float", "lr: float", "beta1: float", "beta2: float", "epsilon: float",
        "grad: T"},
       {},
       {"T: {float, half, bfloat16}", "use_locking: bool = false", "use_nesterov: bool = false"},
       no_output_shape_fn,
       true},
      {"MusaGroupedResourceApplyAdam",
       {"vars: N * resource", "ms: N * resource", "vs: N * resource", "beta1_power: T",
        "beta2_power: T", "lr: T", "beta1: T", "beta2: T", "epsilon: T", "grads: N * Tgrad"},
       {},
       {"N: int >= 1", "T: {float, half, bfloat16, double}",
        "Tgrad: {float, half, bfloat16, double}", "use_locking: bool = false",
        "use_nesterov: bool = false"},
       no_output_shape_fn,
       true},
  };
  return specs;
}

std::vector<KernelSpec> kernel_specs() {
  std::vector<KernelSpec> ks;
  const TF_DataType bn_types[] = {TF_FLOAT, TF_HALF, TF_BFLOAT16};
  for (TF_DataType t : bn_types) {
    // Same compute for every version, as the reference registers them
    // (musa_fused_batchnorm_op.cc:303-325); V2/V3 also fix U = float.
    ks.push_back({"FusedBatchNorm", bn_create<false>, bn_forward_compute,
                  delete_kernel<BnKernel>, {{"T", t}}, {}});
    ks.push_back({"FusedBatchNormV2", bn_create<false>, bn_forward_compute,
                  delete_kernel<BnKernel>, {{"T", t}, {"U", TF_FLOAT}}, {}});
    ks.push_back({"FusedBatchNormV3", bn_create<true>, bn_forward_compute,
                  delete_kernel<BnKernel>, {{"T", t}, {"U", TF_FLOAT}}, {}});
    ks.push_back({"FusedBatchNormGrad", bn_create<false>, bn_grad_compute,
                  delete_kernel<BnKernel>, {{"T", t}}, {}});
    ks.push_back({"FusedBatchNormGradV2", bn_create<false>, bn_grad_compute,
                  delete_kernel<BnKernel>, {{"T", t}, {"U", TF_FLOAT}}, {}});
    ks.push_back({"FusedBatchNormGradV3", bn_create<true>, bn_grad_compute,
                  delete_kernel<BnKernel>, {{"T", t}, {"U", TF_FLOAT}}, {}});
  }
  const std::vector<const char*> adam_host = {"var", "m", "v", "beta1_power", "beta2_power",
                                              "lr", "beta1", "beta2", "epsilon"};
  const std::vector<const char*> scalar_host = {"beta1_power", "beta2_power", "lr",
                                                "beta1", "beta2", "epsilon"};
  const TF_DataType adam_types[] = {TF_FLOAT, TF_HALF, TF_BFLOAT16, TF_DOUBLE};
  for (TF_DataType t : adam_types) {
    ks.push_back({"ResourceApplyAdam", adam_create, adam_compute<false>,
                  delete_kernel<AdamKernel>, {{"T", t}}, adam_host});
    // Reference variables: inputs 0-2 are refs; the forwarded ref output is
    // not set (the C API has no ref outputs), so a graph that reads
    // ApplyAdam's output fails with TensorFlow's missing-output error.
    ks.push_back({"ApplyAdam", adam_create, adam_compute<false>, delete_kernel<AdamKernel>,
                  {{"T", t}}, scalar_host});
    ks.push_back({"MusaGroupedResourceApplyAdam", adam_create, grouped_adam_compute,
                  delete_kernel<AdamKernel>, {{"T", t}, {"Tgrad", t}},
                  {"vars", "ms", "vs", "beta1_power", "beta2_power", "lr", "beta1", "beta2",
                   "epsilon"}});
  }
  // Integer state: the reference registers ResourceApplyAdam (only) for
  // int64 and int32 too (musa_applyadam_op.cc:675-676).
  for (TF_DataType t : {TF_INT64, TF_INT32})
    ks.push_back({"ResourceApplyAdam", adam_create, adam_compute<false>,
                  delete_kernel<AdamKernel>, {{"T", t}}, adam_host});
  for (TF_DataType g : {TF_HALF, TF_BFLOAT16})
    ks.push_back({"MusaGroupedResourceApplyAdam", adam_create, grouped_adam_compute,
                  delete_kernel<AdamKernel>, {{"T", TF_FLOAT}, {"Tgrad", g}},
                  {"vars", "ms", "vs", "beta1_power", "beta2_power", "lr", "beta1", "beta2",
                   "epsilon"}});
  for (TF_DataType g : {TF_FLOAT, TF_HALF, TF_BFLOAT16})
    ks.push_back({"MusaResourceApplyAdamMixed", adam_create, adam_compute<true>,
                  delete_kernel<AdamKernel>, {{"T", g}}, adam_host});
  const TF_DataType ew_types[] = {TF_FLOAT, TF_HALF, TF_BFLOAT16, TF_DOUBLE};
  for (TF_DataType t : ew_types) {
    ks.push_back({"MusaBiasAddRelu", format_create, bias_add_compute<true>,
                  delete_kernel<FormatKernel>, {{"T", t}}, {}});
    ks.push_back({"Relu", plain_create, relu_compute, delete_kernel<FormatKernel>, {{"T", t}}, {}});
    ks.push_back({"ReluGrad", plain_create, relu_grad_compute, delete_kernel<FormatKernel>,
                  {{"T", t}}, {}});
    ks.push_back({"MusaAddV2Relu", plain_create, binary_compute<TFMA_MusaAddV2Relu>,
                  delete_kernel<FormatKernel>, {{"T", t}}, {}});
    ks.push_back({"MusaShiftedAffineMap", plain_create, shifted_affine_map_compute,
                  delete_kernel<FormatKernel>, {{"T", t}}, {}});
  }
  // The stock ops with the reference's dtype lists: AddV2 and the legacy Add
  // (musa_add_op.cc:455-468; bool, whose arithmetic is muDNN's, is left out),
  // Mul (musa_multiply_op.cc:315-323), BiasAdd and BiasAddV1 - BiasAdd
  // without the data_format attr, always NHWC (musa_biasadd_op.cc:67-79).
  for (TF_DataType t : {TF_FLOAT, TF_INT32, TF_INT64, TF_HALF, TF_BFLOAT16, TF_DOUBLE, TF_UINT8}) {
    ks.push_back({"AddV2", plain_create, binary_compute<TFMA_AddV2>, delete_kernel<FormatKernel>,
                  {{"T", t}}, {}});
    ks.push_back({"Add", plain_create, binary_compute<TFMA_AddV2>, delete_kernel<FormatKernel>,
                  {{"T", t}}, {}});
  }
  for (TF_DataType t : {TF_FLOAT, TF_DOUBLE, TF_HALF, TF_BFLOAT16, TF_INT32, TF_INT64}) {
    ks.push_back({"Mul", plain_create, binary_compute<TFMA_Mul>, delete_kernel<FormatKernel>,
                  {{"T", t}}, {}});
    ks.push_back({"BiasAdd", format_create, bias_add_compute<false>,
                  delete_kernel<FormatKernel>, {{"T", t}}, {}});
    ks.push_back({"BiasAddV1", plain_create, bias_add_compute<false>,
                  delete_kernel<FormatKernel>, {{"T", t}}, {}});
  }
  const TF_DataType bag_types[] = {TF_FLOAT, TF_HALF, TF_BFLOAT16, TF_DOUBLE, TF_INT32, TF_INT64};
  for (TF_DataType t : bag_types)
    ks.push_back({"BiasAddGrad", format_create, bias_add_grad_compute,
                  delete_kernel<FormatKernel>, {{"T", t}}, {}});
  return ks;
}

// ===========================================================================
// Graph optimizer.
// ===========================================================================
// Names as NUL-terminated strings from TensorFlow's (value, length) lists.
bool read_names(const TF_GrapplerItem* item, bool preserve, std::vector<std::string>* out,
                TF_Status* s) {
  int num = 0;
  size_t storage = 0;
  if (preserve)
    TF_GetNodesToPreserveListSize(item, &num, &storage, s);
  else
    TF_GetFetchNodesListSize(item, &num, &storage, s);
  if (TF_GetCode(s) != TF_OK) return false;
  std::vector<char*> values(num);
  std::vector<size_t> lengths(num);
  std::vector<char> buf(storage > 0 ? storage : 1);
  if (preserve)
    TF_GetNodesToPreserveList(item, values.data(), lengths.data(), num, buf.data(), storage, s);
  else
    TF_GetFetchNodesList(item, values.data(), lengths.data(), num, buf.data(), storage, s);
  if (TF_GetCode(s) != TF_OK) return false;
  for (int i = 0; i < num; ++i) out->emplace_back(values[i], lengths[i]);
  return true;
}

void free_graph(void* data, size_t) { TFMA_FreeBuffer(data); }

// Patterns switched off through TFMA_DISABLED_FUSION_PATTERNS (a comma list
// of pattern names, as the reference's disabled_fusion_patterns parameter,
// musa_graph_optimizer.cc:5448-5475; a plugin optimizer has no parameters).
const char* disabled_patterns() { return getenv("TFMA_DISABLED_FUSION_PATTERNS"); }

void optimize(void*, const TF_Buffer* graph, const TF_GrapplerItem* item, TF_Buffer* out,
              TF_Status* s) {
  std::vector<std::string> keep;
  if (item && (!read_names(item, true, &keep, s) || !read_names(item, false, &keep, s))) return;
  std::vector<const char*> names;
  for (const std::string& k : keep) names.push_back(k.c_str());
  void* result = nullptr;
  size_t bytes = 0;
  TFMA_Status st;
  const int rc = TFMA_OptimizeGraph(graph->data, graph->length, names.data(),
                                    static_cast<int>(names.size()), kDeviceType,
                                    disabled_patterns(), &result, &bytes, nullptr, &st);
  if (rc != TFMA_OK) {
    set_error(s, static_cast<TF_Code>(rc), "%s", st.message);
    return;
  }
  out->data = result;
  out->length = bytes;
  out->data_deallocator = free_graph;
  set_ok(s);
}

}  // namespace

// ===========================================================================
// Entry points.
// ===========================================================================
extern "C" {

__attribute__((visibility("default"))) void SE_InitPlugin(SE_PlatformRegistrationParams* params,
                                                          TF_Status* status) {
  if (!params) {
    set_error(status, TF_INVALID_ARGUMENT, "null SE_PlatformRegistrationParams");
    return;
  }
  if (params->struct_size < SE_PLATFORM_REGISTRATION_PARAMS_STRUCT_SIZE) {
    set_error(status, TF_INVALID_ARGUMENT,
              "SE_PlatformRegistrationParams struct_size %zu is smaller than %zu",
              params->struct_size, SE_PLATFORM_REGISTRATION_PARAMS_STRUCT_SIZE);
    return;
  }
  if (!params->platform || !params->platform_fns) {
    set_error(status, TF_INVALID_ARGUMENT, "SE_InitPlugin: null platform or platform_fns");
    return;
  }
  if (params->platform->struct_size < SP_PLATFORM_STRUCT_SIZE ||
      params->platform_fns->struct_size < SP_PLATFORM_FNS_STRUCT_SIZE) {
    set_error(status, TF_INVALID_ARGUMENT, "SP_Platform or SP_PlatformFns struct_size too small");
    return;
  }
  params->major_version = SE_MAJOR;
  params->minor_version = SE_MINOR;
  params->patch_version = SE_PATCH;
  params->destroy_platform = destroy_platform;
  params->destroy_platform_fns = destroy_platform_fns;
  SP_Platform* p = params->platform;
  p->struct_size = SP_PLATFORM_STRUCT_SIZE;
  p->name = kPlatformName;
  p->type = kDeviceType;
  p->supports_unified_memory = 0;
  p->use_bfc_allocator = 1;
  p->force_memory_growth = 0;
  SP_PlatformFns* f = params->platform_fns;
  f->struct_size = SP_PLATFORM_FNS_STRUCT_SIZE;
  f->get_device_count = get_device_count;
  f->create_device = create_device;
  f->destroy_device = destroy_device;
  f->create_device_fns = create_device_fns;
  f->destroy_device_fns = destroy_device_fns;
  f->create_stream_executor = create_stream_executor;
  f->destroy_stream_executor = destroy_stream_executor;
  f->create_timer_fns = create_timer_fns;
  f->destroy_timer_fns = destroy_timer_fns;
  set_ok(status);
}

__attribute__((visibility("default"))) void TF_InitKernel(void) {
  TF_Status* s = TF_NewStatus();
  for (const OpSpec& o : op_specs()) {
    if (!register_op(o, s))
      fprintf(stderr, "tfma: op definition %s not registered: %s\n", o.name, TF_Message(s));
    TF_SetStatus(s, TF_OK, "");
  }
  for (const KernelSpec& k : kernel_specs()) {
    if (!register_kernel(k, s))
      fprintf(stderr, "tfma: kernel %s not registered: %s\n", k.op, TF_Message(s));
    TF_SetStatus(s, TF_OK, "");
  }
  TF_DeleteStatus(s);
}

__attribute__((visibility("default"))) void TF_InitGraph(TP_OptimizerRegistrationParams* params,
                                                         TF_Status* status) {
  if (!params) {
    set_error(status, TF_INVALID_ARGUMENT, "null TP_OptimizerRegistrationParams");
    return;
  }
  if (params->struct_size < TP_OPTIMIZER_REGISTRATION_PARAMS_STRUCT_SIZE) {
    set_error(status, TF_INVALID_ARGUMENT,
              "TP_OptimizerRegistrationParams struct_size %zu is smaller than %zu",
              params->struct_size, TP_OPTIMIZER_REGISTRATION_PARAMS_STRUCT_SIZE);
    return;
  }
  if (!params->optimizer || !params->optimizer_configs) {
    set_error(status, TF_INVALID_ARGUMENT, "TF_InitGraph: null optimizer or configs");
    return;
  }
  params->major_version = GO_MAJOR;
  params->minor_version = GO_MINOR;
  params->patch_version = GO_PATCH;
  params->device_type = kDeviceType;
  TP_OptimizerConfigs* c = params->optimizer_configs;
  c->struct_size = TP_OPTIMIZER_CONFIGS_STRUCT_SIZE;
  TP_Optimizer* o = params->optimizer;
  o->struct_size = TP_OPTIMIZER_STRUCT_SIZE;
  o->create_func = nullptr;
  o->optimize_func = optimize;
  o->destroy_func = nullptr;
  set_ok(status);
}

}  // extern "C"

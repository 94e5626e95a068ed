// Internal host-side declarations shared by the op layer and the kernel
// launchers.  Launchers return hipError_t; the op layer turns every failure
// into a TFMA_Status.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "tfma.h"

namespace tfma {

// kI32, kI64, kU8: integer storage for the stock elementwise ops (add and
// multiply, wrapping); no other kernel family takes them.
enum class DType { kF32, kF16, kBF16, kF64, kI32, kI64, kU8 };

inline int DTypeBytes(DType t) {
  switch (t) {
    case DType::kF64: case DType::kI64: return 8;
    case DType::kF32: case DType::kI32: return 4;
    case DType::kU8: return 1;
    default: return 2;
  }
}

// ---------------------------------------------------------------------------
// Kernel launch tracing (TFMA_TraceEnable / TFMA_TraceRead).
// ---------------------------------------------------------------------------
void SetLastKernel(const char* kernel_name);

// Event pair for one launch of `kernel_name` when tracing is on for it (both
// null otherwise).  The launcher hands them to hipExtLaunchKernelGGL, which
// records them as the dispatch's own begin and end, so no marker packets sit
// between kernels; TraceCommit then queues the pair.  The events are never
// destroyed, and are handed out again only after they have completed.
struct TraceEvents {
  hipEvent_t start = nullptr;
  hipEvent_t end = nullptr;
};
TraceEvents TraceTake(const char* kernel_name);
void TraceCommit(const TraceEvents& ev);

// Launches one kernel on `stream` (the arguments of hipLaunchKernelGGL after
// `name`) and records `name` as the last kernel launched.  When tracing is on
// for `name`, HIP events ride on the dispatch itself as its start and end, so
// no marker packets sit between kernels.
#define TFMA_LAUNCH(name, kernel, grid, block, smem, stream, ...)                      \
  do {                                                                                 \
    const char* const tfma_name_ = (name);                                             \
    ::tfma::SetLastKernel(tfma_name_);                                                 \
    const ::tfma::TraceEvents tfma_ev_ = ::tfma::TraceTake(tfma_name_);                \
    hipExtLaunchKernelGGL(kernel, grid, block, smem, stream, tfma_ev_.start, tfma_ev_.end, \
                          0, __VA_ARGS__);                                             \
    ::tfma::TraceCommit(tfma_ev_);                                                     \
  } while (0)

// Plan and cache-mode overrides (TFMA_SetTuningOverride); -1 = not set.
//   kTuneEwNt: elementwise cache mode 0, 1 or 2 instead of the size rule.
//   kTuneBnSliceTw: 0 = fused BN grads unsliced; 4, 8, 16, 32 = sliced in
//     tiles of that many channel vectors.
//   kTuneBnSlicedOverlap: 0 = sliced grads run the plain sliced pass.
//   kTuneBnNchwOwned: 0 = NCHW training keeps the split kernels.
//   kTuneBagFused: 0 = BiasAddGrad runs as two kernels (partials, then finals)
//     instead of one launch.
enum Tune {
  kTuneEwNt,
  kTuneBnSliceTw,
  kTuneBnSlicedOverlap,
  kTuneBnNchwOwned,
  kTuneBagFused,
  kTuneCount
};
int TuneValue(Tune k);
bool SetTune(const char* name, int value);

// Orders launches that share per-device library state (the fused BN
// kernels' counters and epoch regions, BiasAddGrad's tagged slots and static
// scratch): a launch on another stream than the previous one waits for it.
// Launches on one stream are ordered by the stream and carry no event (an
// event on a dispatch delays the next stream operation by ~3 us when the
// stream is otherwise idle).  The first switch of streams on a device
// synchronizes the device once (no event exists yet to wait for, and the
// previous stream may since have been destroyed); from then on every launch
// ends with an event (`own`, or the trace event the launch already carries)
// that the next switch waits for.  A trace event goes back to the tracer's
// pool only once its launch has completed, so waiting for it after it was
// recorded again elsewhere never lets a launch start before the previous
// one ended.  The caller holds the state's mutex.
struct LaunchChain {
  hipEvent_t own = nullptr;    // created on first use
  hipEvent_t chain = nullptr;  // end of the last launch once `multi`
  hipStream_t last_stream = nullptr;
  bool used = false;
  bool multi = false;  // launches from two streams seen on this device

  hipError_t before(hipStream_t s) {
    if (!own) {
      const hipError_t e =
          hipEventCreateWithFlags(&own, hipEventDisableTiming | hipEventReleaseToDevice);
      if (e != hipSuccess) return e;
    }
    if (!used || last_stream == s) return hipSuccess;
    const hipError_t e = multi ? hipStreamWaitEvent(s, chain, 0) : hipDeviceSynchronize();
    multi = true;
    return e;
  }
  // The end event the launch's dispatch carries (null: none).
  hipEvent_t end_event(hipEvent_t trace_end) const { return trace_end ? trace_end : (multi ? own : nullptr); }
  void after(hipStream_t s, hipEvent_t end) {
    chain = end;
    last_stream = s;
    used = true;
  }
};

// Number of compute units of the current device (cached per device).
int DeviceCUs();

// ---------------------------------------------------------------------------
// Adam
// ---------------------------------------------------------------------------
// Host scalars, already in the compute type of T (float for f32/f16/bf16,
// double for f64), with alpha computed the way TF's CPU kernel does.
struct AdamScalars {
  double alpha, beta1, beta2, epsilon, one_minus_beta1, one_minus_beta2;
};

// t: dtype of var/m/v; tg: dtype of grad (tg == t, or t = f32 with a f16 or
// bf16 gradient).
hipError_t LaunchApplyAdam(DType t, DType tg, void* var, void* m, void* v,
                           const void* grad, int64_t n, const AdamScalars& s,
                           bool nesterov, hipStream_t stream);

// Integer ResourceApplyAdam (int32 / int64 var, m, v and grad): the
// reference's generic op chain in T; the scalars as T values (alpha already
// converted from the double the reference computes, 1 - beta in T).
struct IntAdamScalars {
  int64_t alpha, beta1, beta2, eps, omb1, omb2;
};
hipError_t LaunchApplyAdamInt(bool is64, void* var, void* m, void* v, const void* grad,
                              int64_t n, const IntAdamScalars& s, hipStream_t stream);

// One entry of the grouped-Adam tensor table (device memory).
struct AdamTensorEntry {
  void* var;
  void* m;
  void* v;
  const void* grad;
  int64_t n;
  int64_t first_chunk;  // prefix sum of chunks over the preceding tensors
};
constexpr int64_t kGroupedAdamChunk = 8192;  // elements per workgroup chunk

// The tensor table in kernel arguments (launches recorded into a graph):
// kArgTableTensors tensors per launch, 3.1 KB of arguments.
constexpr int kArgTableTensors = 64;
struct AdamArgTable {
  int64_t first_chunk[kArgTableTensors + 1];  // chunk prefix sums; [count] = total
  void* var[kArgTableTensors];
  void* m[kArgTableTensors];
  void* v[kArgTableTensors];
  const void* grad[kArgTableTensors];
  int64_t n[kArgTableTensors];
  int32_t count;
};
hipError_t LaunchGroupedApplyAdamArgs(DType t, DType tg, const AdamTensorEntry* entries,
                                      int n_tensors, const AdamScalars& s, bool nesterov,
                                      hipStream_t stream);

hipError_t LaunchGroupedApplyAdam(DType t, DType tg, const AdamTensorEntry* dev_table,
                                  int n_tensors, int64_t total_chunks,
                                  const AdamScalars& s, bool nesterov,
                                  hipStream_t stream);

// ---------------------------------------------------------------------------
// BiasAddGrad (dt: TFMA_DataType code; x viewed as [outer, c, inner])
// ---------------------------------------------------------------------------
size_t BiasAddGradWorkspaceBytes(int dt, int64_t outer, int64_t c, int64_t inner, int esize);
hipError_t LaunchBiasAddGrad(int dt, const void* x, int64_t outer, int64_t c, int64_t inner,
                             void* out, void* workspace, hipStream_t stream);
// Allocation-free BiasAddGrad: device address, on the current device, of the
// library's static scratch of kBiasAddGradScratchBytes (resolved with
// hipGetSymbolAddress on the device's first call, then cached per device).
constexpr size_t kBiasAddGradScratchBytes = size_t(4) << 20;
hipError_t BiasAddGradScratch(void** ptr);
// BiasAddGrad with the partials in that scratch.  Eager calls on one device
// are chained: a call on another stream than the previous call waits for the
// previous call's end, so overlapping calls do not share the scratch.
hipError_t LaunchBiasAddGradNoAlloc(int dt, const void* x, int64_t outer, int64_t c,
                                    int64_t inner, void* out, hipStream_t stream);
// Zero-fills n bytes with a kernel (capturable, unlike a memset node).
hipError_t LaunchZeroBytes(void* p, int64_t n, hipStream_t stream);
// 16-byte non-temporal streaming copy (bytes a multiple of 16, both pointers
// 16-byte aligned): the measured ceiling bench.py reports.
hipError_t LaunchStreamCopy(void* dst, const void* src, int64_t bytes, hipStream_t stream);

// ---------------------------------------------------------------------------
// Elementwise
// ---------------------------------------------------------------------------
// kReluGrad: a = gradients, b = features (TF's gradients * (features > 0)).
enum class EwOp { kAdd, kAddRelu, kMul, kMulAdd, kRelu, kReluGrad };

// How an input of an elementwise kernel maps a flat output index i to its
// own flat index: kFull: i; kScalar: 0; kPeriodic: (i / inner) % period.
enum class BcastMode { kFull, kScalar, kPeriodic };
struct BcastOperand {
  const void* data;
  BcastMode mode;
  int64_t inner;
  int64_t period;
};

// out[i] = op(a[i], b[i], c[i]) for i < n.  Operands past the op's arity are
// ignored.  a is the "value" input; all operands have dtype t.  Above 2^31
// elements the range runs in chunks whose length is a multiple of every
// periodic operand's cycle (inner * period); ElementwiseFlatOk says whether
// that is possible (a cycle below 2^31 elements), else use the strided path.
bool ElementwiseFlatOk(int64_t n, const BcastOperand& a, const BcastOperand& b,
                       const BcastOperand& c);
hipError_t LaunchElementwise(DType t, EwOp op, int64_t n,
                             const BcastOperand& a, const BcastOperand& b,
                             const BcastOperand& c, void* out,
                             hipStream_t stream);

// General strided broadcast fallback (rank <= 8): strides are in elements,
// 0 on broadcast dimensions.
struct StridedShape {
  int ndims;
  int64_t dims[TFMA_MAX_DIMS];
  int64_t stride_a[TFMA_MAX_DIMS];
  int64_t stride_b[TFMA_MAX_DIMS];
  int64_t stride_c[TFMA_MAX_DIMS];
};
hipError_t LaunchElementwiseStrided(DType t, EwOp op, int64_t n,
                                    const void* a, const void* b,
                                    const void* c, const StridedShape& shape,
                                    void* out, hipStream_t stream);

// ---------------------------------------------------------------------------
// Fused batch norm
// ---------------------------------------------------------------------------
struct BnGeometry {
  bool nhwc;
  int64_t n, c, h, w;  // logical NCHW sizes
  int64_t rows;        // elements per channel = n*h*w
};

// Scratch bytes needed by the BN kernels for this geometry and dtype.
size_t BnWorkspaceBytes(DType t, const BnGeometry& g);

struct BnFwdArgs {
  const void* x;
  const float* scale;
  const float* offset;
  const float* mean_in;  // running mean (exponential average / inference)
  const float* var_in;   // running variance
  float epsilon;
  float exp_avg_factor;
  bool is_training;
  void* y;
  float* batch_mean;
  float* batch_var;
  float* saved_mean;
  float* saved_var;
  float* reserve3;  // 0-d scalar, may be null
};
hipError_t LaunchBnForward(DType t, const BnGeometry& g, const BnFwdArgs& a,
                           void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

struct BnGradArgs {
  const void* dy;
  const void* x;
  const float* scale;
  const float* saved_mean;
  const float* saved_var;
  float epsilon;
  bool is_training;
  void* dx;
  float* scale_backprop;
  float* offset_backprop;
  float* reserve4;
  int64_t reserve4_n;
  float* reserve5;
  int64_t reserve5_n;
};
hipError_t LaunchBnGrad(DType t, const BnGeometry& g, const BnGradArgs& a,
                        void* workspace, size_t workspace_bytes,
                        hipStream_t stream);
// Reads (and with `reset` clears) the current device's give-up word after a
// device synchronize.
hipError_t BnBarrierTimedOut(bool reset, bool* timed_out);
// Whether a fused launch on the current device gave up one of its waits and
// has not been reported yet (no device synchronization: the kernel writes
// the word to pinned host memory).  On true, *epoch is that launch's epoch
// and the report is consumed.
bool BnPendingGiveUp(unsigned* epoch);
// Plan of the calling thread's last FusedBatchNorm launch.
TFMA_FusedBatchNormPlan BnLastPlan();
// Copies the fused kernel's phase stamps to host memory after a device
// synchronize (hipErrorNotSupported unless built with -DTFMA_BN_STAMPS).
hipError_t BnStamps(void* host, size_t bytes);

}  // namespace tfma

/*
 * tfma.h — C ABI of the MI355X (gfx950) fused data-parallel kernel library.
 *
 * This is the drop-in boundary for the hot path of
 * MooreThreads/tensorflow_musa_extension: FusedBatchNormV3 /
 * FusedBatchNormGradV3, ResourceApplyAdam and a multi-tensor (grouped) Adam,
 * and the elementwise chains BiasAdd+Relu, AddV2+Relu and Mul+Add.
 *
 * Each entry point is what a TensorFlow PluggableDevice kernel's compute
 * callback (registered through TF_NewKernelBuilder in TF_InitKernel) would
 * call after it has resolved its inputs, allocated its outputs and fetched
 * its stream: plain pointers, shapes and dtypes, a hipStream_t passed as
 * void*, and a status object that mirrors TF_Status.  Nothing here uses
 * torch or TensorFlow types.
 *
 * Conventions
 *  - Codes in TFMA_Code have the numeric values of TF_Code
 *    (tensorflow/c/tf_status.h); dtypes in TFMA_DataType have the numeric
 *    values of TF_DataType (tensorflow/c/tf_datatype.h).
 *  - Every entry point returns the status code and also stores it, with a
 *    message, in *status.  No entry point throws or aborts.
 *  - Work is enqueued on `stream` and the call returns without waiting for
 *    the device (no host synchronisation), as the reference's ops do on the
 *    TF-provided stream.
 *  - Outputs are allocated by the caller with the shapes the op's shape
 *    function gives (TF's allocate_output); the library checks them and
 *    reports INVALID_ARGUMENT on a mismatch.
 *  - Scratch memory comes from the caller (the `workspace` arguments, sized
 *    by the *WorkspaceBytes queries), as TF kernels take it from
 *    allocate_temp.
 */
#ifndef TFMA_H_
#define TFMA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TFMA_MAX_DIMS 8

/* Same numeric values as TF_Code. */
typedef enum TFMA_Code {
  TFMA_OK = 0,
  TFMA_CANCELLED = 1,
  TFMA_UNKNOWN = 2,
  TFMA_INVALID_ARGUMENT = 3,
  TFMA_NOT_FOUND = 5,
  TFMA_RESOURCE_EXHAUSTED = 8,
  TFMA_FAILED_PRECONDITION = 9,
  TFMA_OUT_OF_RANGE = 11,
  TFMA_UNIMPLEMENTED = 12,
  TFMA_INTERNAL = 13,
  TFMA_UNAVAILABLE = 14
} TFMA_Code;

/* Same numeric values as TF_DataType. */
typedef enum TFMA_DataType {
  TFMA_FLOAT = 1,
  TFMA_DOUBLE = 2,
  TFMA_INT32 = 3,
  TFMA_UINT8 = 4,
  TFMA_INT64 = 9,
  TFMA_BFLOAT16 = 14,
  TFMA_HALF = 19
} TFMA_DataType;

/* A dense, row-major tensor: device memory unless an entry point says the
 * argument is host memory (TF's HostMemory inputs). */
typedef struct TFMA_Tensor {
  void* data;
  int32_t dtype;  /* TFMA_DataType */
  int32_t ndims;  /* 0 .. TFMA_MAX_DIMS */
  int64_t dims[TFMA_MAX_DIMS];
} TFMA_Tensor;

/* Mirrors TF_Status: a code and a NUL-terminated message. */
typedef struct TFMA_Status {
  int32_t code;
  char message[500];
} TFMA_Status;

/* ---------------------------------------------------------------------------
 * Library / device
 * ------------------------------------------------------------------------- */

/* Version string of the library, e.g. "tfma 0.1 gfx950". */
const char* TFMA_Version(void);

/* Number of visible HIP devices; 0 (and TFMA_OK) when no driver or device is
 * present.  Replaces plugin_get_device_count
 * (reference: musa_ext/mu/musa_se_plugin.cc:855-880), including its
 * "no driver -> zero devices, OK" behaviour. */
int TFMA_GetDeviceCount(int* count, TFMA_Status* status);

/* ---------------------------------------------------------------------------
 * FusedBatchNormV3 / FusedBatchNormGradV3
 * Replaces MusaFusedBatchNormOp<T>::Compute and
 * MusaFusedBatchNormGradOp<T>::Compute
 * (reference: musa_ext/kernels/nn/musa_fused_batchnorm_op.cc:42-182, 206-295;
 * registrations :303-325) together with the BN helper kernels
 * (musa_ext/kernels/nn/musa_fused_batchnorm_kernel.mu:16-56).
 *
 * x/y/y_backprop/x_backprop: rank-4 T tensors, T in {FLOAT, HALF, BFLOAT16};
 * data_format "NHWC" or "NCHW".  scale, offset, mean, variance and every
 * statistics output: rank-1 FLOAT tensors of length C (U = float).
 * reserve_space_3: 0-d FLOAT scalar, written with 0 (reference :59-62,
 * :100-104).  reserve_space_4/5 of the grad: FLOAT tensors of any length
 * (the reference allocates [C], :220-223), filled with zeros.
 * The fused (persistent, NHWC training) path keeps the values its workgroups
 * hand to each other - partial sums and per-channel coefficients, tagged
 * with a per-launch epoch - in library-owned device memory (24 KB per CU,
 * allocated and zeroed on the device's first fused launch: run one eagerly
 * before capturing a graph); the caller's workspace serves the other paths.
 * ------------------------------------------------------------------------- */

/* Scratch bytes FusedBatchNormV3 / FusedBatchNormGradV3 need for this x. */
int TFMA_FusedBatchNormWorkspaceBytes(const TFMA_Tensor* x,
                                      const char* data_format,
                                      size_t* bytes, TFMA_Status* status);

int TFMA_FusedBatchNormV3(void* stream, const TFMA_Tensor* x,
                          const TFMA_Tensor* scale, const TFMA_Tensor* offset,
                          const TFMA_Tensor* mean, const TFMA_Tensor* variance,
                          float epsilon, float exponential_avg_factor,
                          const char* data_format, int is_training,
                          TFMA_Tensor* y, TFMA_Tensor* batch_mean,
                          TFMA_Tensor* batch_variance,
                          TFMA_Tensor* reserve_space_1,
                          TFMA_Tensor* reserve_space_2,
                          TFMA_Tensor* reserve_space_3, void* workspace,
                          size_t workspace_bytes, TFMA_Status* status);

int TFMA_FusedBatchNormGradV3(
    void* stream, const TFMA_Tensor* y_backprop, const TFMA_Tensor* x,
    const TFMA_Tensor* scale, const TFMA_Tensor* reserve_space_1,
    const TFMA_Tensor* reserve_space_2, const TFMA_Tensor* reserve_space_3,
    float epsilon, const char* data_format, int is_training,
    TFMA_Tensor* x_backprop, TFMA_Tensor* scale_backprop,
    TFMA_Tensor* offset_backprop, TFMA_Tensor* reserve_space_4,
    TFMA_Tensor* reserve_space_5, void* workspace, size_t workspace_bytes,
    TFMA_Status* status);

/* ---------------------------------------------------------------------------
 * ResourceApplyAdam
 * Replaces MusaResourceApplyAdamOp<T>::Compute
 * (reference: musa_ext/kernels/training/musa_applyadam_op.cc:130-416,
 * registration :645-682) and its fp32 kernel
 * (musa_ext/kernels/training/musa_apply_sparse_adam_kernel.mu:140-169).
 *
 * var, m, v: the variables' device tensors, updated in place; grad: device
 * tensor; all the same shape and dtype T in {FLOAT, HALF, BFLOAT16, DOUBLE,
 * INT32, INT64}.  beta1_power .. epsilon: 0-d HOST tensors of dtype T
 * (HostMemory inputs).  Floating T: TF-CPU's update in T.  Integer T: the
 * reference's generic op chain (:224-246, 300-408) in T with two's-complement
 * wrap - alpha from the scalars in double, converted to T (truncation; T's
 * minimum for NaN or out of range), m = m*b1 + g*(1-b1),
 * v = v*b2 + (g*g)*(1-b2), var -= (m / (isqrt(v) + eps)) * alpha with the
 * exact integer square root (0 for v <= 0) and truncating division
 * (x / 0 = 0, MIN / -1 = MIN); use_nesterov has no integer form.
 * A NULL var/m/v data pointer with a non-empty shape is an uninitialised
 * variable (FAILED_PRECONDITION).  use_locking serialises calls that touch
 * the same var/m/v memory through this library (locks taken in address
 * order, reference :138-156).
 * ------------------------------------------------------------------------- */
int TFMA_ResourceApplyAdam(void* stream, TFMA_Tensor* var, TFMA_Tensor* m,
                           TFMA_Tensor* v, const TFMA_Tensor* beta1_power,
                           const TFMA_Tensor* beta2_power,
                           const TFMA_Tensor* lr, const TFMA_Tensor* beta1,
                           const TFMA_Tensor* beta2,
                           const TFMA_Tensor* epsilon, const TFMA_Tensor* grad,
                           int use_locking, int use_nesterov,
                           TFMA_Status* status);

/* Mixed-precision Adam: fp32 var/m/v (T = float state) with a float, half or
 * bfloat16 gradient and float host scalars.  Same op name, inputs, attrs and
 * error messages as the reference's MusaResourceApplyAdamMixed
 * (musa_ext/kernels/training/musa_applyadam_mixed_op.cc:125-302, registered
 * :265-300; kernel musa_applyadam_mixed_kernel.mu:55-103).  The update is
 * bit-identical to TF's Cast(grad, float) followed by the fp32
 * ResourceApplyAdam, the pair the reference's Cast-folding rewrite replaces
 * (musa_ext/graph/fusion/adam_mixed_fusion.cc:93-216); the reference's own
 * kernel uses a different operation order and a double-precision alpha. */
int TFMA_MusaResourceApplyAdamMixed(void* stream, TFMA_Tensor* var, TFMA_Tensor* m,
                                    TFMA_Tensor* v, const TFMA_Tensor* beta1_power,
                                    const TFMA_Tensor* beta2_power, const TFMA_Tensor* lr,
                                    const TFMA_Tensor* beta1, const TFMA_Tensor* beta2,
                                    const TFMA_Tensor* epsilon, const TFMA_Tensor* grad,
                                    int use_locking, int use_nesterov, TFMA_Status* status);

/* Multi-tensor Adam: N independent ResourceApplyAdam updates with shared
 * host scalars in one launch; each element's result is bit-identical to
 * TFMA_ResourceApplyAdam on that tensor.  No reference op exists; it follows
 * the reference's grouped optimizer op
 * MusaGroupedResourceApplyGradientDescentMixed
 * (reference: musa_ext/kernels/training/musa_applygradientdescent_op.cc:
 * 305-448, kernel musa_applygradientdescent_kernel.mu:31-105) with inputs
 * vars/ms/vs/grads: N tensors each.  With fp32 vars the grads may all be
 * half or bfloat16 instead (attr Tgrad, as the reference op's T/Tgrad pair):
 * each tensor then updates as TFMA_MusaResourceApplyAdamMixed.  The
 * per-launch table (the tensor entries and a tensor index per 8192-element
 * chunk; its size depends on the tensors' element counts, hence `vars`)
 * lives in `workspace` (TFMA_GroupedApplyAdamWorkspaceBytes); the library
 * uploads it on the stream, so the workspace must stay allocated until the
 * launch has run.  The library also keeps device copies of the last few
 * tables per device: a call with the same tensors as an earlier one uploads
 * nothing and leaves the workspace untouched.  Recorded into a graph (stream
 * capture), the call puts the table in the kernel arguments instead (64
 * tensors per launch), so every replay updates the tensors of the recorded
 * call; the workspace is then not used. */
int TFMA_GroupedApplyAdamWorkspaceBytes(int n, const TFMA_Tensor* vars,
                                        size_t* bytes, TFMA_Status* status);

int TFMA_GroupedResourceApplyAdam(
    void* stream, int n, TFMA_Tensor* vars, TFMA_Tensor* ms, TFMA_Tensor* vs,
    const TFMA_Tensor* grads, const TFMA_Tensor* beta1_power,
    const TFMA_Tensor* beta2_power, const TFMA_Tensor* lr,
    const TFMA_Tensor* beta1, const TFMA_Tensor* beta2,
    const TFMA_Tensor* epsilon, int use_locking, int use_nesterov,
    void* workspace, size_t workspace_bytes, TFMA_Status* status);

/* ---------------------------------------------------------------------------
 * Elementwise ops and fused chains, T in {FLOAT, HALF, BFLOAT16}.
 * Stock ops replace MusaBiasAddOp (musa_ext/kernels/nn/musa_biasadd_op.cc:
 * 10-82), MusaReluOp (musa_ext/kernels/nn/musa_relu_op.cc:10-60),
 * MusaAddOp (musa_ext/kernels/math/musa_add_op.cc:379-470) and
 * MusaMultiplyOp (musa_ext/kernels/math/musa_multiply_op.cc:248-324).
 * Binary ops follow TF broadcasting (BCast); `z`/`output` must have the
 * broadcast shape.
 *
 * dtypes, as the reference registers them: every op takes FLOAT, HALF,
 * BFLOAT16 and DOUBLE.  TFMA_AddV2 (which also serves TF's legacy `Add`,
 * musa_add_op.cc:455-470) takes INT32, INT64 and UINT8; TFMA_Mul INT32 and
 * INT64 (musa_multiply_op.cc:315-325); TFMA_BiasAdd (which also serves
 * `BiasAddV1` with data_format NULL = "NHWC", musa_biasadd_op.cc:67-80) INT32
 * and INT64.  Integer add and multiply wrap modulo 2^bits (two's
 * complement), as TF's CPU kernels do.  The reference's bool Add is not
 * provided (its semantics are muDNN's, unpinned).
 * ------------------------------------------------------------------------- */
int TFMA_BiasAdd(void* stream, const TFMA_Tensor* value,
                 const TFMA_Tensor* bias, const char* data_format,
                 TFMA_Tensor* output, TFMA_Status* status);
int TFMA_Relu(void* stream, const TFMA_Tensor* features,
              TFMA_Tensor* activations, TFMA_Status* status);
int TFMA_AddV2(void* stream, const TFMA_Tensor* x, const TFMA_Tensor* y,
               TFMA_Tensor* z, TFMA_Status* status);
int TFMA_Mul(void* stream, const TFMA_Tensor* x, const TFMA_Tensor* y,
             TFMA_Tensor* z, TFMA_Status* status);

/* ReluGrad: backprops = gradients * (features > 0), a multiply as in TF's
 * CPU kernel (a NaN or infinite gradient at features <= 0 gives NaN; a
 * negative one gives -0).  Replaces MusaReluGradOp<T>::Compute
 * (reference: musa_ext/kernels/nn/musa_relu_grad_op.cc:10-61, registered
 * :51-57 for float, half, bfloat16), including its same-shape check and
 * message.  Also takes double. */
int TFMA_ReluGrad(void* stream, const TFMA_Tensor* gradients, const TFMA_Tensor* features,
                  TFMA_Tensor* backprops, TFMA_Status* status);

/* BiasAddGrad: output[c] = sum of out_backprop over every dimension except
 * the channel one (the last for "NHWC", dimension 1 for "NCHW" when rank >=
 * 2).  Replaces MusaBiasAddGradOp<T>::Compute
 * (reference: musa_ext/kernels/nn/musa_biasadd_grad_op.cc:24-110,
 * registered :112-123) for T in {FLOAT, HALF, BFLOAT16, DOUBLE, INT32,
 * INT64}: rank 1 is returned as is (:50-58), an empty reduction gives zeros
 * (:64-69).  Half and bfloat16 accumulate in float (as TF's CPU kernel);
 * integers wrap.  The sum runs in a fixed order (deterministic): per-group
 * partials, then per-channel finals over them in group order.  Eager float,
 * half and bfloat16 calls run both in one launch whose last workgroups take
 * the finals, with the partials in library-owned device memory (4 MiB per
 * device, allocated and zeroed on the device's first such call; calls on one
 * device are chained across streams); the other dtypes, launches under
 * stream capture and inputs with more partials than that memory holds run
 * two kernels with the partials in `workspace`
 * (TFMA_BiasAddGradWorkspaceBytes).  Both forms give the same bits. */
int TFMA_BiasAddGradWorkspaceBytes(const TFMA_Tensor* out_backprop, const char* data_format,
                                   size_t* bytes, TFMA_Status* status);
int TFMA_BiasAddGrad(void* stream, const TFMA_Tensor* out_backprop, const char* data_format,
                     TFMA_Tensor* output, void* workspace, size_t workspace_bytes,
                     TFMA_Status* status);

/* Allocation-free BiasAddGrad.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same inputs, result and
 * errors as TFMA_BiasAddGrad, but the per-group partials live in a static
 * device array of the library (4 MiB per GPU, held until the process
 * ends) instead of a caller workspace; the call allocates nothing.  An input
 * whose partials need more (TFMA_BiasAddGradWorkspaceBytes > 4 MiB, i.e.
 * more than about a million channels) is INVALID_ARGUMENT.  All calls on one
 * GPU share that array: calls that overlap on one GPU (concurrent streams)
 * race and must be serialized by the caller. */
int TFMA_BiasAddGradNoAlloc(void* stream, const TFMA_Tensor* out_backprop,
                            const char* data_format, TFMA_Tensor* output,
                            TFMA_Status* status);

/* Fused Relu(BiasAdd(value, bias)).  No live reference op: the reference
 * runs BiasAdd then Relu (musa_biasadd_op.cc:10-70, musa_relu_op.cc:10-62);
 * its only fused kernel, BiasAddReluKernel
 * (musa_ext/kernels/fusion/musa_linear_relu_kernel.mu:41-91), has no
 * caller.  Result is bitwise equal to the unfused pair. */
int TFMA_MusaBiasAddRelu(void* stream, const TFMA_Tensor* value,
                         const TFMA_Tensor* bias, const char* data_format,
                         TFMA_Tensor* output, TFMA_Status* status);

/* Fused Relu(AddV2(x, y)) with TF broadcasting.  No reference op: the
 * reference runs MusaAddOp then MusaReluOp (musa_add_op.cc:388-459).
 * Bitwise equal to the unfused pair. */
int TFMA_MusaAddV2Relu(void* stream, const TFMA_Tensor* x,
                       const TFMA_Tensor* y, TFMA_Tensor* z,
                       TFMA_Status* status);

/* Fused Mul+Add: output = data_left * mask + sliced_var_right, each input
 * broadcast to the output (rank <= 8), rounded after the multiply and after
 * the add as the unfused Mul -> AddV2 pair is.  Same op name, inputs and
 * broadcast shape rule as MusaShiftedAffineMap
 * (musa_ext/kernels/fusion/musa_shifted_affine_map_op.cc:108-262). */
int TFMA_MusaShiftedAffineMap(void* stream, const TFMA_Tensor* data_left,
                              const TFMA_Tensor* mask,
                              const TFMA_Tensor* sliced_var_right,
                              TFMA_Tensor* output, TFMA_Status* status);

/* ---------------------------------------------------------------------------
 * Graph rewrite (host only).  Replaces the reference's fusion pass:
 * FusionPattern match/apply/priority (musa_ext/graph/fusion/
 * fusion_pattern_manager.h:54-82) driven by OptimizeFusion
 * (musa_ext/mu/optimizer/musa_graph_optimizer.cc:5843-5994), and the grouped
 * optimizer rewrite (musa_graph_optimizer.cc:2014-2120), which the reference
 * has for SGD only and this pass does for ResourceApplyAdam.
 *
 * Input and output are serialized tensorflow.GraphDef protos (what a
 * TF_InitGraph optimizer's optimize_func receives and returns in TF_Buffers).
 * Patterns, in priority order:
 *   "MusaBiasAddRelu"       Relu(BiasAdd(x, b))     -> MusaBiasAddRelu(x, b)
 *   "MusaAddV2Relu"         Relu(AddV2|Add(x, y))   -> MusaAddV2Relu(x, y)
 *   "MusaShiftedAffineMap"  AddV2|Add(Mul(x, a), b) -> MusaShiftedAffineMap(x, a, b)
 *   "MusaResourceApplyAdamMixed"  ResourceApplyAdam<float> whose grad is
 *       Cast<half|bfloat16 -> float>(g) -> MusaResourceApplyAdamMixed (T = the
 *       Cast's SrcT) reading g; the Cast is removed when nothing else reads
 *       it (reference pattern MusaAdamMixedFusion, adam_mixed_fusion.cc:93-216,
 *       priority 40).
 *   "MusaGroupedResourceApplyAdam"  >= 2 ResourceApplyAdam or
 *       MusaResourceApplyAdamMixed nodes sharing device, state and gradient
 *       dtypes, use_locking, use_nesterov and the six scalar inputs, none
 *       depending on another, distinct var/m/v ->
 *       MusaGroupedResourceApplyAdam(vars N, ms N, vs N, beta1_power,
 *       beta2_power, lr, beta1, beta2, epsilon, grads N; attrs N, T (state),
 *       Tgrad, use_locking, use_nesterov).
 * The reference's names MusaShiftedAffineMapFusion and MusaAdamMixedFusion
 * are accepted in disabled_patterns as well.
 * A fused node keeps the name, device and control inputs of the node it
 * replaces and gains the absorbed node's control inputs; the absorbed node
 * must have that node as its only data consumer, the same device and T
 * (float, half or bfloat16), and must not be fetched.
 *
 * fetch_nodes: names ("name" or "name:port") that must survive; may be NULL.
 * device_filter: rewrite only nodes whose device string contains it (the
 *   reference matches on "MUSA"); NULL or "" = every node.
 * disabled_patterns: comma-separated pattern names to skip (the reference's
 *   disabled_fusion_patterns parameter, musa_graph_optimizer.cc:5448-5475).
 * On success *optimized is a malloc'd buffer the caller frees with
 * TFMA_FreeBuffer.  A malformed GraphDef is TFMA_INVALID_ARGUMENT.
 * ------------------------------------------------------------------------- */
typedef struct TFMA_GraphRewriteStats {
  int32_t bias_add_relu;      /* fused nodes created per pattern */
  int32_t add_v2_relu;
  int32_t mul_add;
  int32_t adam_groups;        /* grouped Adam nodes created */
  int32_t adam_grouped_nodes; /* Adam nodes they replaced */
  int32_t adam_mixed;         /* Cast folded into MusaResourceApplyAdamMixed */
} TFMA_GraphRewriteStats;

int TFMA_OptimizeGraph(const void* graph_def, size_t graph_def_bytes,
                       const char* const* fetch_nodes, int num_fetch,
                       const char* device_filter, const char* disabled_patterns,
                       void** optimized, size_t* optimized_bytes,
                       TFMA_GraphRewriteStats* stats, TFMA_Status* status);
void TFMA_FreeBuffer(void* buffer);

/* ---------------------------------------------------------------------------
 * Kernel timing.  No reference counterpart (the reference removed its kernel
 * timing macros and points to external profilers).  When a kernel whose name
 * contains `name_substr` is launched by this library, HIP events on the
 * launch stream bracket it (the fused BatchNorm kernels carry them as the
 * dispatch's own start and end events, hipExtLaunchKernelGGL; the others get
 * event records right before and after the launch); TFMA_TraceRead returns
 * the summed event time and the launch count.  TFMA_TraceEnable(NULL)
 * switches tracing off.  Not thread-safe against concurrent launches.
 * ------------------------------------------------------------------------- */
int TFMA_TraceEnable(const char* name_substr, TFMA_Status* status);
int TFMA_TraceRead(double* total_ms, int64_t* launches, TFMA_Status* status);

/* Device-to-device copy of `bytes` (a multiple of 16; both pointers 16-byte
 * aligned, else INVALID_ARGUMENT) by a plain streaming kernel: 16-byte
 * non-temporal loads and stores, grid-stride.  A measuring stick, not an op:
 * bench.py reports its rate as the stream-copy ceiling the kernels' rates sit
 * beside.  No reference counterpart. */
int TFMA_StreamCopy(void* stream, void* dst, const void* src, uint64_t bytes,
                    TFMA_Status* status);

/* The fused BatchNorm kernel assumes its workgroups (one or two per CU) are
 * all resident at once; a wave waiting for another workgroup's partials or
 * coefficients gives up after a bounded spin (~0.5 s), which only happens
 * when another persistent kernel holds compute units the grid needs (another
 * process's, or a graph replay overlapping an eager fused launch).  Such a
 * launch writes NaN statistics and outputs for the channels concerned and
 * stores its epoch in a host-visible word; the next FusedBatchNormV3 /
 * FusedBatchNormGradV3 call on the device then returns TFMA_INTERNAL instead
 * of launching (once per such launch; no device synchronization).
 * This query: *timed_out = 1 if any fused launch on the current device gave
 * up since the last reset; reset != 0 clears it.  Waits for the device to go
 * idle (hipDeviceSynchronize) first: a diagnostic, not for hot loops.
 * No reference counterpart: the reference's BatchNorm kernels have no
 * grid-wide wait. */
int TFMA_FusedBatchNormBarrierTimedOut(int32_t* timed_out, int32_t reset, TFMA_Status* status);

/* Launch plan of the calling thread's last FusedBatchNormV3 /
 * FusedBatchNormGradV3 call (for tests that check which path ran).
 * fused = 1: the persistent kernel ran with `workgroups` workgroups over
 * row_groups x channel_tiles; dynamic_rows > 0: each thread's lowest
 * dynamic_rows streamed phase-3 rows were handed out in chunks of
 * dynamic_chunk rows; register_rows / lds_rows: rows per thread kept on chip;
 * slices > 1: each workgroup ran channel_tiles / slices tiles at a time, one
 * whole two-phase pass per slice (1: all tiles at once).
 * fused = 2: the NCHW kernel with one workgroup per channel ran
 * (workgroups = channel_tiles = C).
 * fused = 0: the reduce / finalize / apply kernels ran.  No reference
 * counterpart. */
typedef struct TFMA_FusedBatchNormPlan {
  int32_t fused;
  int32_t workgroups;
  int64_t row_groups;
  int32_t channel_tiles;
  int32_t dynamic_rows;
  int32_t dynamic_chunk;
  int32_t register_rows;
  int32_t lds_rows;
  int32_t slices;
} TFMA_FusedBatchNormPlan;
int TFMA_FusedBatchNormLastPlan(TFMA_FusedBatchNormPlan* plan, TFMA_Status* status);

/* Name of the last kernel this library launched on the calling thread (for
 * tests that check which path an op took). */
const char* TFMA_LastKernelName(void);

/* Plan and cache-mode overrides, for tests and measurements (no reference
 * counterpart).  `value` -1 restores the library's own choice.
 *   "ew_nt"             elementwise cache mode: 0 plain loads and stores,
 *                       1 non-temporal loads of full-size operands, 2 also
 *                       non-temporal row operands and stores (default: by
 *                       size).
 *   "bn_slice_tw"       fused BatchNorm gradients: 0 never sliced; 4, 8, 16
 *                       or 32 sliced (where such a plan exists, at most 8
 *                       slices) in tiles of that many channel vectors.
 *   "bn_sliced_overlap" 0: sliced gradients run the plain sliced pass
 *                       instead of hiding each slice's hand-off.
 *   "bn_nchw_owned"     0: NCHW training keeps the split kernels instead of
 *                       one workgroup per channel.
 *   "bag_fused"         0: BiasAddGrad runs as two kernels (partials, then
 *                       per-channel finals) instead of one launch.
 * Each starts from the environment variable TFMA_<NAME in upper case>,
 * read once, at the library's first query of any override; after that the
 * launch paths read one atomic value (no getenv on the hot path).  An
 * unknown name is INVALID_ARGUMENT.
 *
 * Environment variables read once by the library (diagnostics; not needed
 * in normal use): TFMA_BN_FORCE_GIVE_UP=1 makes every eager fused BatchNorm
 * launch give up its grid-wide waits after a short spin (exercises the
 * co-residency error path: NaN outputs, then INTERNAL, see
 * TFMA_FusedBatchNormBarrierTimedOut); TFMA_BN_EPOCH_START=<n> starts the
 * fused launches' epoch counter at n (runs launches across its wrap);
 * TFMA_BN_FUSED=0 disables the fused BatchNorm kernels; TFMA_BN_DYN_PCT,
 * TFMA_BN_DYN_CHUNK, TFMA_BN_TARGET_WGS and TFMA_EW_BLOCKS_PER_CU change
 * launch shapes for measurements; TFMA_COPY_THREADS sizes the host copy
 * pool. */
int TFMA_SetTuningOverride(const char* name, int32_t value, TFMA_Status* status);

/* Phase timestamps of the fused NHWC BatchNorm kernel, for measurement
 * builds only (no reference counterpart): with the library built with
 * -DTFMA_BN_STAMPS, lane 0 of every wave of the last fused launches records
 * a 100 MHz clock (s_memrealtime) at 7 points; this call synchronizes the
 * device and copies `count` values, laid out [workgroup][wave 0..7][slot
 * 0..7] for workgroups below 1024.  Slots: 0 entry, 1 phase-1 sums done,
 * 2 partials published, 3 finals done, 4 coefficients in, 5 static phase-3
 * rows written, 6 dynamic tail done, 7 the XCD the wave ran on.  A
 * workgroup's values are those of the last launch that ran it (a sliced
 * launch: its last slice).  UNIMPLEMENTED in a normal build. */
int TFMA_FusedBatchNormStamps(uint64_t* stamps, uint64_t count, TFMA_Status* status);

/* ---------------------------------------------------------------------------
 * Host data path of the stream executor: what the SP_StreamExecutor copy,
 * dependency and callback slots forward to (TF: memcpy_htod /
 * sync_memcpy_htod, memcpy_dtoh / sync_memcpy_dtoh, create_stream_dependency,
 * host_callback).  All act on the current device.
 * ------------------------------------------------------------------------- */

/* Host -> device copy of `size` bytes.  A pageable source is staged through
 * pinned blocks in 4 MiB chunks (the host copy of one chunk overlaps the DMA
 * of the previous one); the call returns once the source has been read, so
 * the caller may reuse it at once, also when sync == 0.  A pinned source is
 * copied directly; a device source becomes a device-to-device copy.
 * sync != 0: on the null stream, returns when the copy is done (`stream` is
 * ignored).  Replaces plugin_se_memcpy_htod / plugin_se_sync_memcpy_htod and
 * MemcpyHtoDWithPinnedBounce (reference: musa_ext/mu/musa_se_plugin.cc:
 * 127-211, 621-641, 730-747); errors: null pointers with size > 0 ->
 * INVALID_ARGUMENT ("null host pointer for src in memcpy_htod"), HIP
 * failures -> INTERNAL. */
int TFMA_MemcpyHtoD(void* stream, void* device_dst, const void* host_src, uint64_t size,
                    int32_t sync, TFMA_Status* status);

/* Device -> host copy.  sync != 0 into pageable memory: staged in 4 MiB
 * chunks (DMA of one chunk overlaps the host copy of the previous one);
 * otherwise one hipMemcpyAsync on `stream` (the null stream when sync).
 * Replaces plugin_se_memcpy_dtoh / plugin_se_sync_memcpy_dtoh
 * (musa_se_plugin.cc:599-619, 712-728). */
int TFMA_MemcpyDtoH(void* stream, void* host_dst, const void* device_src, uint64_t size,
                    int32_t sync, TFMA_Status* status);

/* Work enqueued on `dependent` after this call waits for the work enqueued
 * on `other` before it.  Events come from a per-device pool and are reused
 * once the recorded work has run (the reference creates and later destroys
 * one per call).  Replaces plugin_se_create_stream_dependency
 * (musa_se_plugin.cc:365-432); null stream -> INVALID_ARGUMENT. */
int TFMA_CreateStreamDependency(void* dependent, void* other, TFMA_Status* status);

/* Runs fn(arg) on a host thread once the work enqueued on `stream` before it
 * has completed (hipLaunchHostFunc).  Replaces plugin_se_host_callback
 * (musa_se_plugin.cc:808-835; the TF adapter wraps SE_StatusCallbackFn). */
int TFMA_HostCallback(void* stream, void (*fn)(void*), void* arg, TFMA_Status* status);

/* Staging pool of the current device: pinned blocks allocated so far, host
 * allocations, reuses of a free block, and entries (blocks or dependency
 * events) still waiting for their work.  No reference counterpart (the
 * reference logs these counters, pinned_memory_pool.cc:120-160). */
int TFMA_StagingPoolStats(uint64_t* blocks, uint64_t* host_allocs, uint64_t* reuses,
                          uint64_t* pending, TFMA_Status* status);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* TFMA_H_ */

/*
 * tf_c_api.h - the parts of TensorFlow's public C API that the PluggableDevice
 * adapter (tf_plugin.cc) uses, restated from TensorFlow's published headers:
 *   tensorflow/c/tf_status.h, tf_datatype.h, tf_tensor.h, c_api.h (TF_Buffer)
 *   tensorflow/c/kernels.h, kernels_experimental.h, ops.h
 *   tensorflow/c/experimental/stream_executor/stream_executor.h
 *   tensorflow/c/experimental/grappler/grappler.h
 * Names, signatures, enum values and struct member order follow those headers
 * as of TensorFlow 2.15 (the newest version the reference builds against,
 * build.sh:17).  TensorFlow is not installed in this image, so the struct
 * layouts here are not checked against a TensorFlow build: a maintainer who
 * builds against a real TensorFlow should include its headers instead
 * (define TFMA_USE_TENSORFLOW_HEADERS) and the adapter compiles unchanged.
 * Every struct carries struct_size, which TensorFlow and the plugin check
 * against the sizes below.
 */
#ifndef TFMA_TF_C_API_H_
#define TFMA_TF_C_API_H_

#ifdef TFMA_USE_TENSORFLOW_HEADERS
#include "tensorflow/c/c_api.h"
#include "tensorflow/c/experimental/grappler/grappler.h"
#include "tensorflow/c/experimental/stream_executor/stream_executor.h"
#include "tensorflow/c/kernels.h"
#include "tensorflow/c/kernels_experimental.h"
#include "tensorflow/c/ops.h"
#else

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TF_OFFSET_OF_END(TYPE, MEMBER) (offsetof(TYPE, MEMBER) + sizeof(((TYPE*)0)->MEMBER))

typedef unsigned char TF_Bool;

/* ---- tf_status.h ------------------------------------------------------- */
typedef struct TF_Status TF_Status;
typedef enum TF_Code {
  TF_OK = 0,
  TF_CANCELLED = 1,
  TF_UNKNOWN = 2,
  TF_INVALID_ARGUMENT = 3,
  TF_DEADLINE_EXCEEDED = 4,
  TF_NOT_FOUND = 5,
  TF_ALREADY_EXISTS = 6,
  TF_PERMISSION_DENIED = 7,
  TF_UNAUTHENTICATED = 16,
  TF_RESOURCE_EXHAUSTED = 8,
  TF_FAILED_PRECONDITION = 9,
  TF_ABORTED = 10,
  TF_OUT_OF_RANGE = 11,
  TF_UNIMPLEMENTED = 12,
  TF_INTERNAL = 13,
  TF_UNAVAILABLE = 14,
  TF_DATA_LOSS = 15
} TF_Code;
extern TF_Status* TF_NewStatus(void);
extern void TF_DeleteStatus(TF_Status*);
extern void TF_SetStatus(TF_Status* s, TF_Code code, const char* msg);
extern TF_Code TF_GetCode(const TF_Status* s);
extern const char* TF_Message(const TF_Status* s);

/* ---- tf_datatype.h ----------------------------------------------------- */
typedef enum TF_DataType {
  TF_FLOAT = 1,
  TF_DOUBLE = 2,
  TF_INT32 = 3,
  TF_UINT8 = 4,
  TF_INT16 = 5,
  TF_INT8 = 6,
  TF_STRING = 7,
  TF_COMPLEX64 = 8,
  TF_INT64 = 9,
  TF_BOOL = 10,
  TF_QINT8 = 11,
  TF_QUINT8 = 12,
  TF_QINT32 = 13,
  TF_BFLOAT16 = 14,
  TF_QINT16 = 15,
  TF_QUINT16 = 16,
  TF_UINT16 = 17,
  TF_COMPLEX128 = 18,
  TF_HALF = 19,
  TF_RESOURCE = 20,
  TF_VARIANT = 21,
  TF_UINT32 = 22,
  TF_UINT64 = 23
} TF_DataType;

/* ---- tf_tensor.h ------------------------------------------------------- */
typedef struct TF_Tensor TF_Tensor;
extern void TF_DeleteTensor(TF_Tensor*);
extern TF_DataType TF_TensorType(const TF_Tensor*);
extern int TF_NumDims(const TF_Tensor*);
extern int64_t TF_Dim(const TF_Tensor* tensor, int dim_index);
extern size_t TF_TensorByteSize(const TF_Tensor*);
extern void* TF_TensorData(const TF_Tensor*);
extern int64_t TF_TensorElementCount(const TF_Tensor* tensor);

typedef struct TF_AllocatorAttributes {
  size_t struct_size;
  TF_Bool on_host;
} TF_AllocatorAttributes;
#define TF_ALLOCATOR_ATTRIBUTES_STRUCT_SIZE TF_OFFSET_OF_END(TF_AllocatorAttributes, on_host)

/* ---- c_api.h: TF_Buffer ------------------------------------------------ */
typedef struct TF_Buffer {
  const void* data;
  size_t length;
  void (*data_deallocator)(void* data, size_t length);
} TF_Buffer;

/* ---- stream_executor.h ------------------------------------------------- */
#define SE_MAJOR 0
#define SE_MINOR 0
#define SE_PATCH 1

typedef struct SP_Stream_st* SP_Stream;
typedef struct SP_Event_st* SP_Event;
typedef struct SP_Timer_st* SP_Timer;
typedef void (*SE_StatusCallbackFn)(void* const, TF_Status* const);

typedef struct SP_TimerFns {
  size_t struct_size;
  void* ext;
  uint64_t (*nanoseconds)(SP_Timer timer);
} SP_TimerFns;
#define SP_TIMER_FNS_STRUCT_SIZE TF_OFFSET_OF_END(SP_TimerFns, nanoseconds)

typedef struct SP_AllocatorStats {
  size_t struct_size;
  int64_t num_allocs;
  int64_t bytes_in_use;
  int64_t peak_bytes_in_use;
  int64_t largest_alloc_size;
  int8_t has_bytes_limit;
  int64_t bytes_limit;
  int64_t bytes_reserved;
  int64_t peak_bytes_reserved;
  int8_t has_bytes_reservable_limit;
  int64_t bytes_reservable_limit;
  int64_t largest_free_block_bytes;
} SP_AllocatorStats;
#define SP_ALLOCATORSTATS_STRUCT_SIZE TF_OFFSET_OF_END(SP_AllocatorStats, largest_free_block_bytes)

typedef enum SE_EventStatus {
  SE_EVENT_UNKNOWN,
  SE_EVENT_ERROR,
  SE_EVENT_PENDING,
  SE_EVENT_COMPLETE,
} SE_EventStatus;

typedef struct SP_DeviceMemoryBase {
  size_t struct_size;
  void* ext;
  void* opaque;
  uint64_t size;
  uint64_t payload;
} SP_DeviceMemoryBase;
#define SP_DEVICE_MEMORY_BASE_STRUCT_SIZE TF_OFFSET_OF_END(SP_DeviceMemoryBase, payload)

typedef struct SP_Device {
  size_t struct_size;
  void* ext;
  int32_t ordinal;
  void* device_handle;
  const char* hardware_name;
  const char* device_vendor;
  const char* pci_bus_id;
} SP_Device;
#define SP_DEVICE_STRUCT_SIZE TF_OFFSET_OF_END(SP_Device, pci_bus_id)

typedef struct SE_CreateDeviceParams {
  size_t struct_size;
  void* ext;
  int32_t ordinal;
  SP_Device* device;
} SE_CreateDeviceParams;
#define SE_CREATE_DEVICE_PARAMS_STRUCT_SIZE TF_OFFSET_OF_END(SE_CreateDeviceParams, device)

typedef struct SP_DeviceFns {
  size_t struct_size;
  void* ext;
  int32_t (*get_numa_node)(const SP_Device* device);
  int64_t (*get_memory_bandwidth)(const SP_Device* device);
  double (*get_gflops)(const SP_Device* device);
} SP_DeviceFns;
#define SP_DEVICE_FNS_STRUCT_SIZE TF_OFFSET_OF_END(SP_DeviceFns, get_gflops)

typedef struct SE_CreateDeviceFnsParams {
  size_t struct_size;
  void* ext;
  SP_DeviceFns* device_fns;
} SE_CreateDeviceFnsParams;
#define SE_CREATE_DEVICE_FNS_PARAMS_STRUCT_SIZE \
  TF_OFFSET_OF_END(SE_CreateDeviceFnsParams, device_fns)

typedef struct SP_StreamExecutor {
  size_t struct_size;
  void* ext;
  void (*allocate)(const SP_Device* device, uint64_t size, int64_t memory_space,
                   SP_DeviceMemoryBase* mem);
  void (*deallocate)(const SP_Device* device, SP_DeviceMemoryBase* memory);
  void* (*host_memory_allocate)(const SP_Device* device, uint64_t size);
  void (*host_memory_deallocate)(const SP_Device* device, void* mem);
  void* (*unified_memory_allocate)(const SP_Device* device, uint64_t bytes);
  void (*unified_memory_deallocate)(const SP_Device* device, void* location);
  TF_Bool (*get_allocator_stats)(const SP_Device* device, SP_AllocatorStats* stats);
  TF_Bool (*device_memory_usage)(const SP_Device* device, int64_t* free, int64_t* total);
  void (*create_stream)(const SP_Device* device, SP_Stream* stream, TF_Status* status);
  void (*destroy_stream)(const SP_Device* device, SP_Stream stream);
  void (*create_stream_dependency)(const SP_Device* device, SP_Stream dependent,
                                   SP_Stream other, TF_Status* status);
  void (*get_stream_status)(const SP_Device* device, SP_Stream stream, TF_Status* status);
  void (*create_event)(const SP_Device* device, SP_Event* event, TF_Status* status);
  void (*destroy_event)(const SP_Device* device, SP_Event event);
  SE_EventStatus (*get_event_status)(const SP_Device* device, SP_Event event);
  void (*record_event)(const SP_Device* device, SP_Stream stream, SP_Event event,
                       TF_Status* status);
  void (*wait_for_event)(const SP_Device* const device, SP_Stream stream, SP_Event event,
                         TF_Status* const status);
  void (*create_timer)(const SP_Device* device, SP_Timer* timer, TF_Status* status);
  void (*destroy_timer)(const SP_Device* device, SP_Timer timer);
  void (*start_timer)(const SP_Device* device, SP_Stream stream, SP_Timer timer,
                      TF_Status* status);
  void (*stop_timer)(const SP_Device* device, SP_Stream stream, SP_Timer timer,
                     TF_Status* status);
  void (*memcpy_dtoh)(const SP_Device* device, SP_Stream stream, void* host_dst,
                      const SP_DeviceMemoryBase* device_src, uint64_t size, TF_Status* status);
  void (*memcpy_htod)(const SP_Device* device, SP_Stream stream, SP_DeviceMemoryBase* device_dst,
                      const void* host_src, uint64_t size, TF_Status* status);
  void (*memcpy_dtod)(const SP_Device* device, SP_Stream stream, SP_DeviceMemoryBase* device_dst,
                      const SP_DeviceMemoryBase* device_src, uint64_t size, TF_Status* status);
  void (*sync_memcpy_dtoh)(const SP_Device* device, void* host_dst,
                           const SP_DeviceMemoryBase* device_src, uint64_t size,
                           TF_Status* status);
  void (*sync_memcpy_htod)(const SP_Device* device, SP_DeviceMemoryBase* device_dst,
                           const void* host_src, uint64_t size, TF_Status* status);
  void (*sync_memcpy_dtod)(const SP_Device* device, SP_DeviceMemoryBase* device_dst,
                           const SP_DeviceMemoryBase* device_src, uint64_t size,
                           TF_Status* status);
  void (*block_host_for_event)(const SP_Device* device, SP_Event event, TF_Status* status);
  void (*block_host_until_done)(const SP_Device* device, SP_Stream stream, TF_Status* status);
  void (*synchronize_all_activity)(const SP_Device* device, TF_Status* status);
  void (*mem_zero)(const SP_Device* device, SP_Stream stream, SP_DeviceMemoryBase* location,
                   uint64_t size, TF_Status* status);
  void (*memset)(const SP_Device* device, SP_Stream stream, SP_DeviceMemoryBase* location,
                 uint8_t pattern, uint64_t size, TF_Status* status);
  void (*memset32)(const SP_Device* device, SP_Stream stream, SP_DeviceMemoryBase* location,
                   uint32_t pattern, uint64_t size, TF_Status* status);
  TF_Bool (*host_callback)(const SP_Device* device, SP_Stream stream,
                           SE_StatusCallbackFn callback_fn, void* callback_arg);
} SP_StreamExecutor;
#define SP_STREAMEXECUTOR_STRUCT_SIZE TF_OFFSET_OF_END(SP_StreamExecutor, host_callback)

typedef struct SE_CreateStreamExecutorParams {
  size_t struct_size;
  void* ext;
  SP_StreamExecutor* stream_executor;
} SE_CreateStreamExecutorParams;
#define SE_CREATE_STREAM_EXECUTOR_PARAMS_STRUCT_SIZE \
  TF_OFFSET_OF_END(SE_CreateStreamExecutorParams, stream_executor)

typedef struct SP_Platform {
  size_t struct_size;
  void* ext;
  const char* name;
  const char* type;
  TF_Bool supports_unified_memory;
  TF_Bool use_bfc_allocator;
  TF_Bool force_memory_growth;
} SP_Platform;
#define SP_PLATFORM_STRUCT_SIZE TF_OFFSET_OF_END(SP_Platform, force_memory_growth)

typedef struct SP_PlatformFns {
  size_t struct_size;
  void* ext;
  void (*get_device_count)(const SP_Platform* platform, int* device_count, TF_Status* status);
  void (*create_device)(const SP_Platform* platform, SE_CreateDeviceParams* params,
                        TF_Status* status);
  void (*destroy_device)(const SP_Platform* platform, SP_Device* device);
  void (*create_device_fns)(const SP_Platform* platform, SE_CreateDeviceFnsParams* params,
                            TF_Status* status);
  void (*destroy_device_fns)(const SP_Platform* platform, SP_DeviceFns* device_fns);
  void (*create_stream_executor)(const SP_Platform* platform,
                                 SE_CreateStreamExecutorParams* params, TF_Status* status);
  void (*destroy_stream_executor)(const SP_Platform* platform,
                                  SP_StreamExecutor* stream_executor);
  void (*create_timer_fns)(const SP_Platform* platform, SP_TimerFns* timer, TF_Status* status);
  void (*destroy_timer_fns)(const SP_Platform* platform, SP_TimerFns* timer_fns);
} SP_PlatformFns;
#define SP_PLATFORM_FNS_STRUCT_SIZE TF_OFFSET_OF_END(SP_PlatformFns, destroy_timer_fns)

typedef struct SE_PlatformRegistrationParams {
  size_t struct_size;
  void* ext;
  int32_t major_version;
  int32_t minor_version;
  int32_t patch_version;
  SP_Platform* platform;
  SP_PlatformFns* platform_fns;
  void (*destroy_platform)(SP_Platform* platform);
  void (*destroy_platform_fns)(SP_PlatformFns* platform_fns);
} SE_PlatformRegistrationParams;
#define SE_PLATFORM_REGISTRATION_PARAMS_STRUCT_SIZE \
  TF_OFFSET_OF_END(SE_PlatformRegistrationParams, destroy_platform_fns)

/* ---- kernels.h --------------------------------------------------------- */
typedef struct TF_KernelBuilder TF_KernelBuilder;
typedef struct TF_OpKernelConstruction TF_OpKernelConstruction;
typedef struct TF_OpKernelContext TF_OpKernelContext;

extern TF_KernelBuilder* TF_NewKernelBuilder(const char* op_name, const char* device_name,
                                             void* (*create_func)(TF_OpKernelConstruction*),
                                             void (*compute_func)(void*, TF_OpKernelContext*),
                                             void (*delete_func)(void*));
extern void TF_KernelBuilder_TypeConstraint(TF_KernelBuilder* kernel_builder,
                                            const char* attr_name, const TF_DataType type,
                                            TF_Status* status);
extern void TF_KernelBuilder_HostMemory(TF_KernelBuilder* kernel_builder, const char* arg_name);
extern void TF_KernelBuilder_Priority(TF_KernelBuilder* kernel_builder, int32_t priority_number);
extern void TF_RegisterKernelBuilder(const char* kernel_name, TF_KernelBuilder* builder,
                                     TF_Status* status);
extern void TF_DeleteKernelBuilder(TF_KernelBuilder* builder);

extern SP_Stream TF_GetStream(TF_OpKernelContext* ctx, TF_Status* status);
extern int TF_NumInputs(TF_OpKernelContext* ctx);
extern int TF_NumOutputs(TF_OpKernelContext* ctx);
extern void TF_GetInput(TF_OpKernelContext* ctx, int i, TF_Tensor** tensor, TF_Status* status);
extern void TF_SetOutput(TF_OpKernelContext* ctx, int i, const TF_Tensor* tensor,
                         TF_Status* status);
extern void TF_OpKernelContext_Failure(TF_OpKernelContext* ctx, TF_Status* status);
extern TF_Tensor* TF_AllocateOutput(TF_OpKernelContext* context, int index, TF_DataType dtype,
                                    const int64_t* dims, int num_dims, size_t len,
                                    TF_Status* status);
extern TF_Tensor* TF_ForwardInputOrAllocateOutput(TF_OpKernelContext* context,
                                                  const int* candidate_input_indices,
                                                  int num_candidate_input_indices,
                                                  int output_index, const int64_t* output_dims,
                                                  int output_num_dims, int* forwarded_input,
                                                  TF_Status* status);
extern TF_Tensor* TF_AllocateTemp(TF_OpKernelContext* context, TF_DataType dtype,
                                  const int64_t* dims, int num_dims,
                                  TF_AllocatorAttributes* alloc_attrs, TF_Status* status);

extern void TF_OpKernelConstruction_GetAttrSize(TF_OpKernelConstruction* ctx,
                                                const char* attr_name, int32_t* list_size,
                                                int32_t* total_size, TF_Status* status);
extern void TF_OpKernelConstruction_GetAttrType(TF_OpKernelConstruction* ctx,
                                                const char* attr_name, TF_DataType* val,
                                                TF_Status* status);
extern void TF_OpKernelConstruction_GetAttrInt32(TF_OpKernelConstruction* ctx,
                                                 const char* attr_name, int32_t* val,
                                                 TF_Status* status);
extern void TF_OpKernelConstruction_GetAttrFloat(TF_OpKernelConstruction* ctx,
                                                 const char* attr_name, float* val,
                                                 TF_Status* status);
extern void TF_OpKernelConstruction_GetAttrBool(TF_OpKernelConstruction* ctx,
                                                const char* attr_name, TF_Bool* val,
                                                TF_Status* status);
extern void TF_OpKernelConstruction_GetAttrString(TF_OpKernelConstruction* ctx,
                                                  const char* attr_name, char* val,
                                                  size_t max_length, TF_Status* status);
extern bool TF_OpKernelConstruction_HasAttr(TF_OpKernelConstruction* ctx,
                                            const char* attr_name, TF_Status* status);
extern void TF_OpKernelConstruction_Failure(TF_OpKernelConstruction* ctx, TF_Status* status);

/* ---- kernels_experimental.h -------------------------------------------- */
typedef struct TF_VariableInputLockHolder TF_VariableInputLockHolder;
extern void TF_MaybeLockVariableInput(TF_OpKernelContext* ctx, int* inputs, size_t len,
                                      bool isVariantType, bool sparse,
                                      void (*copyFunc)(TF_OpKernelContext* ctx,
                                                       TF_Tensor* source, TF_Tensor* dest),
                                      TF_VariableInputLockHolder** lockHolder,
                                      TF_Status* status);
extern void TF_GetInputTensorFromVariable(TF_OpKernelContext* ctx, int input, bool lock_held,
                                          bool isVariantType, bool sparse,
                                          void (*copyFunc)(TF_OpKernelContext* ctx,
                                                           TF_Tensor* source, TF_Tensor* dest),
                                          TF_Tensor** out, TF_Status* status);
extern void TF_ReleaseVariableInputLockHolder(TF_VariableInputLockHolder* lockHolder);

/* ---- ops.h ------------------------------------------------------------- */
typedef struct TF_OpDefinitionBuilder TF_OpDefinitionBuilder;
typedef struct TF_ShapeInferenceContext TF_ShapeInferenceContext;
typedef struct TF_ShapeHandle TF_ShapeHandle;
typedef struct TF_DimensionHandle TF_DimensionHandle;

extern TF_OpDefinitionBuilder* TF_NewOpDefinitionBuilder(const char* op_name);
extern void TF_RegisterOpDefinition(TF_OpDefinitionBuilder* builder, TF_Status* status);
extern void TF_DeleteOpDefinitionBuilder(TF_OpDefinitionBuilder* builder);
extern void TF_OpDefinitionBuilderAddAttr(TF_OpDefinitionBuilder* builder, const char* attr_spec);
extern void TF_OpDefinitionBuilderAddInput(TF_OpDefinitionBuilder* builder,
                                           const char* input_spec);
extern void TF_OpDefinitionBuilderAddOutput(TF_OpDefinitionBuilder* builder,
                                            const char* output_spec);
extern void TF_OpDefinitionBuilderSetIsCommutative(TF_OpDefinitionBuilder* builder,
                                                   bool is_commutative);
extern void TF_OpDefinitionBuilderSetIsStateful(TF_OpDefinitionBuilder* builder,
                                                bool is_stateful);
extern void TF_OpDefinitionBuilderSetShapeInferenceFunction(
    TF_OpDefinitionBuilder* builder,
    void (*shape_inference_func)(TF_ShapeInferenceContext* ctx, TF_Status* status));

extern int64_t TF_ShapeInferenceContextNumInputs(TF_ShapeInferenceContext* ctx);
extern TF_ShapeHandle* TF_NewShapeHandle(void);
extern void TF_DeleteShapeHandle(TF_ShapeHandle* handle);
extern TF_DimensionHandle* TF_NewDimensionHandle(void);
extern void TF_DeleteDimensionHandle(TF_DimensionHandle* handle);
extern void TF_ShapeInferenceContextGetInput(TF_ShapeInferenceContext* ctx, int i,
                                             TF_ShapeHandle* handle, TF_Status* status);
extern void TF_ShapeInferenceContextSetOutput(TF_ShapeInferenceContext* ctx, int i,
                                              TF_ShapeHandle* handle, TF_Status* status);
extern void TF_ShapeInferenceContextSetUnknownShape(TF_ShapeInferenceContext* ctx,
                                                    TF_Status* status);
extern int TF_ShapeInferenceContextRankKnown(TF_ShapeInferenceContext* ctx,
                                             TF_ShapeHandle* handle);
extern int64_t TF_ShapeInferenceContextRank(TF_ShapeInferenceContext* ctx,
                                            TF_ShapeHandle* handle);
extern void TF_ShapeInferenceContextDim(TF_ShapeInferenceContext* ctx,
                                        TF_ShapeHandle* shape_handle, int64_t i,
                                        TF_DimensionHandle* result);
extern int TF_DimensionHandleValueKnown(TF_DimensionHandle* dim_handle);
extern int64_t TF_DimensionHandleValue(TF_DimensionHandle* dim_handle);

/* ---- grappler.h -------------------------------------------------------- */
#define GO_MAJOR 0
#define GO_MINOR 0
#define GO_PATCH 1

typedef enum TF_TriState {
  TF_TriState_Default = 0,
  TF_TriState_Off,
  TF_TriState_On,
} TF_TriState;

typedef struct TF_GrapplerItem TF_GrapplerItem;

typedef struct TP_OptimizerConfigs {
  size_t struct_size;
  void* ext;
  TF_TriState disable_model_pruning;
  TF_TriState implementation_selector;
  TF_TriState function_optimization;
  TF_TriState common_subgraph_elimination;
  TF_TriState arithmetic_optimization;
  TF_TriState debug_stripper;
  TF_TriState constant_folding;
  TF_TriState shape_optimization;
  TF_TriState auto_mixed_precision;
  TF_TriState auto_mixed_precision_onednn_bfloat16;
  TF_TriState auto_mixed_precision_mkl;
  TF_TriState pin_to_host_optimization;
  TF_TriState layout_optimizer;
  TF_TriState remapping;
  TF_TriState loop_optimization;
  TF_TriState dependency_optimization;
  TF_TriState auto_parallel;
  TF_TriState memory_optimization;
  TF_TriState scoped_allocator_optimization;
} TP_OptimizerConfigs;
#define TP_OPTIMIZER_CONFIGS_STRUCT_SIZE \
  TF_OFFSET_OF_END(TP_OptimizerConfigs, scoped_allocator_optimization)

typedef struct TP_Optimizer {
  size_t struct_size;
  void* ext;
  void* (*create_func)(void);
  void (*optimize_func)(void*, const TF_Buffer*, const TF_GrapplerItem*, TF_Buffer*,
                        TF_Status*);
  void (*destroy_func)(void*);
} TP_Optimizer;
#define TP_OPTIMIZER_STRUCT_SIZE TF_OFFSET_OF_END(TP_Optimizer, destroy_func)

typedef struct TP_OptimizerRegistrationParams {
  size_t struct_size;
  void* ext;
  int32_t major_version;
  int32_t minor_version;
  int32_t patch_version;
  const char* device_type;
  TP_OptimizerConfigs* optimizer_configs;
  TP_Optimizer* optimizer;
} TP_OptimizerRegistrationParams;
#define TP_OPTIMIZER_REGISTRATION_PARAMS_STRUCT_SIZE \
  TF_OFFSET_OF_END(TP_OptimizerRegistrationParams, optimizer)

extern void TF_GetFetchNodesListSize(const TF_GrapplerItem* item, int* num_values,
                                     size_t* storage_size, TF_Status* status);
extern void TF_GetFetchNodesList(const TF_GrapplerItem* item, char** values, size_t* lengths,
                                 int num_values, void* storage, size_t storage_size,
                                 TF_Status* status);
extern void TF_GetNodesToPreserveListSize(const TF_GrapplerItem* item, int* num_values,
                                          size_t* storage_size, TF_Status* status);
extern void TF_GetNodesToPreserveList(const TF_GrapplerItem* item, char** values,
                                      size_t* lengths, int num_values, void* storage,
                                      size_t storage_size, TF_Status* status);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* TFMA_USE_TENSORFLOW_HEADERS */
#endif  /* TFMA_TF_C_API_H_ */

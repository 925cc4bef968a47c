/*
 * Test double of the ONNX Runtime C API: the subset the custom-op layer under
 * xmetai-onnx-plugins_amd/csrc/ort uses, with the public names, argument
 * order and semantics of onnxruntime_c_api.h (status objects, custom-op
 * domains, kernel info attributes, kernel context inputs/outputs/stream/
 * scratch, tensor type and shape).  The struct layouts are this double's own,
 * so a library built against it runs only under ort_double.cpp, never under
 * ONNX Runtime.  Test infrastructure only.
 */
#ifndef XM_TEST_ORT_DOUBLE_C_API_H_
#define XM_TEST_ORT_DOUBLE_C_API_H_

#include <stddef.h>
#include <stdint.h>

#define ORT_API_VERSION 17
#define ORT_API_CALL

#ifdef __cplusplus
extern "C" {
#endif

/* ONNX TensorProto element types */
typedef enum ONNXTensorElementDataType {
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED = 0,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT = 1,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8 = 2,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT8 = 3,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT16 = 4,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT16 = 5,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32 = 6,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64 = 7,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_STRING = 8,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_BOOL = 9,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16 = 10,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_DOUBLE = 11,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT32 = 12,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT64 = 13,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_COMPLEX64 = 14,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_COMPLEX128 = 15,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16 = 16
} ONNXTensorElementDataType;

typedef enum OrtErrorCode {
    ORT_OK = 0,
    ORT_FAIL = 1,
    ORT_INVALID_ARGUMENT = 2,
    ORT_RUNTIME_EXCEPTION = 6,
    ORT_NOT_IMPLEMENTED = 9
} OrtErrorCode;

typedef enum OrtCustomOpInputOutputCharacteristic {
    INPUT_OUTPUT_REQUIRED = 0,
    INPUT_OUTPUT_OPTIONAL,
    INPUT_OUTPUT_VARIADIC
} OrtCustomOpInputOutputCharacteristic;

typedef struct OrtStatus OrtStatus;
typedef struct OrtValue OrtValue;
typedef struct OrtKernelInfo OrtKernelInfo;
typedef struct OrtKernelContext OrtKernelContext;
typedef struct OrtCustomOpDomain OrtCustomOpDomain;
typedef struct OrtSessionOptions OrtSessionOptions;
typedef struct OrtTensorTypeAndShapeInfo OrtTensorTypeAndShapeInfo;
typedef struct OrtMemoryInfo OrtMemoryInfo;

typedef struct OrtAllocator {
    uint32_t version;
    void *(ORT_API_CALL *Alloc)(struct OrtAllocator *self, size_t size);
    void(ORT_API_CALL *Free)(struct OrtAllocator *self, void *p);
    const OrtMemoryInfo *(ORT_API_CALL *Info)(const struct OrtAllocator *self);
} OrtAllocator;

struct OrtApi;

typedef struct OrtCustomOp {
    uint32_t version;
    void *(ORT_API_CALL *CreateKernel)(const struct OrtCustomOp *op, const struct OrtApi *api, const OrtKernelInfo *info);
    const char *(ORT_API_CALL *GetName)(const struct OrtCustomOp *op);
    const char *(ORT_API_CALL *GetExecutionProviderType)(const struct OrtCustomOp *op);
    ONNXTensorElementDataType(ORT_API_CALL *GetInputType)(const struct OrtCustomOp *op, size_t index);
    size_t(ORT_API_CALL *GetInputTypeCount)(const struct OrtCustomOp *op);
    ONNXTensorElementDataType(ORT_API_CALL *GetOutputType)(const struct OrtCustomOp *op, size_t index);
    size_t(ORT_API_CALL *GetOutputTypeCount)(const struct OrtCustomOp *op);
    void(ORT_API_CALL *KernelCompute)(void *op_kernel, OrtKernelContext *context);
    void(ORT_API_CALL *KernelDestroy)(void *op_kernel);
    OrtCustomOpInputOutputCharacteristic(ORT_API_CALL *GetInputCharacteristic)(const struct OrtCustomOp *op, size_t index);
    OrtCustomOpInputOutputCharacteristic(ORT_API_CALL *GetOutputCharacteristic)(const struct OrtCustomOp *op, size_t index);
} OrtCustomOp;

typedef struct OrtApi {
    OrtStatus *(ORT_API_CALL *CreateStatus)(OrtErrorCode code, const char *msg);
    OrtErrorCode(ORT_API_CALL *GetErrorCode)(const OrtStatus *status);
    const char *(ORT_API_CALL *GetErrorMessage)(const OrtStatus *status);
    void(ORT_API_CALL *ReleaseStatus)(OrtStatus *status);
    OrtStatus *(ORT_API_CALL *CreateCustomOpDomain)(const char *domain, OrtCustomOpDomain **out);
    OrtStatus *(ORT_API_CALL *CustomOpDomain_Add)(OrtCustomOpDomain *domain, const OrtCustomOp *op);
    OrtStatus *(ORT_API_CALL *AddCustomOpDomain)(OrtSessionOptions *options, OrtCustomOpDomain *domain);
    OrtStatus *(ORT_API_CALL *KernelInfoGetAttribute_float)(const OrtKernelInfo *info, const char *name, float *out);
    OrtStatus *(ORT_API_CALL *KernelInfoGetAttribute_int64)(const OrtKernelInfo *info, const char *name, int64_t *out);
    OrtStatus *(ORT_API_CALL *KernelContext_GetInputCount)(const OrtKernelContext *context, size_t *out);
    OrtStatus *(ORT_API_CALL *KernelContext_GetOutputCount)(const OrtKernelContext *context, size_t *out);
    OrtStatus *(ORT_API_CALL *KernelContext_GetInput)(const OrtKernelContext *context, size_t index, const OrtValue **out);
    OrtStatus *(ORT_API_CALL *KernelContext_GetOutput)(OrtKernelContext *context, size_t index, const int64_t *dim_values,
                                                        size_t dim_count, OrtValue **out);
    OrtStatus *(ORT_API_CALL *KernelContext_GetGPUComputeStream)(const OrtKernelContext *context, void **out);
    OrtStatus *(ORT_API_CALL *KernelContext_GetAllocator)(const OrtKernelContext *context, const OrtMemoryInfo *mem_info,
                                                           OrtAllocator **out);
    OrtStatus *(ORT_API_CALL *KernelContext_GetScratchBuffer)(const OrtKernelContext *context,
                                                               const OrtMemoryInfo *mem_info, size_t count_or_bytes,
                                                               void **out);
    void(ORT_API_CALL *ReleaseAllocator)(OrtAllocator *allocator);
    OrtStatus *(ORT_API_CALL *GetTensorTypeAndShape)(const OrtValue *value, OrtTensorTypeAndShapeInfo **out);
    OrtStatus *(ORT_API_CALL *GetDimensionsCount)(const OrtTensorTypeAndShapeInfo *info, size_t *out);
    OrtStatus *(ORT_API_CALL *GetDimensions)(const OrtTensorTypeAndShapeInfo *info, int64_t *dim_values,
                                             size_t dim_values_length);
    OrtStatus *(ORT_API_CALL *GetTensorElementType)(const OrtTensorTypeAndShapeInfo *info, ONNXTensorElementDataType *out);
    void(ORT_API_CALL *ReleaseTensorTypeAndShapeInfo)(OrtTensorTypeAndShapeInfo *info);
    OrtStatus *(ORT_API_CALL *GetTensorMutableData)(OrtValue *value, void **out);
    OrtStatus *(ORT_API_CALL *GetTensorMemoryInfo)(const OrtValue *value, const OrtMemoryInfo **out);
} OrtApi;

typedef struct OrtApiBase {
    const OrtApi *(ORT_API_CALL *GetApi)(uint32_t version);
    const char *(ORT_API_CALL *GetVersionString)(void);
} OrtApiBase;

#ifdef __cplusplus
}
#endif

#endif /* XM_TEST_ORT_DOUBLE_C_API_H_ */

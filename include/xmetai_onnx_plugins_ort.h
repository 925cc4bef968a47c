/*
 * xmetai_onnx_plugins_ort.h — ONNX Runtime custom-op entry point.
 *
 * libxmetai_onnx_plugins_ort.so registers the domain "xmetai_plugins" with
 * the operators SelectiveScanFn, Mamba3SisoFn, GatedDeltaNet2Fn (ROCm
 * execution provider, gfx950 kernels through xmetai_recurrent.h) and
 * SoftmaxCPU (CPU execution provider), in that order.  Exported graphs that
 * use these node types load unchanged.
 *
 * Reference: csrc/register_op.cpp:11-41 (same symbol, same domain, same
 * operator order; the only change is the GPU execution provider string,
 * "ROCMExecutionProvider" instead of "CUDAExecutionProvider").
 *
 * Loaded by ONNX Runtime through SessionOptions.register_custom_ops_library
 * (Python) or RegisterCustomOpsLibrary_V2 / the C API equivalent.  Returns
 * NULL on success, else the first failing OrtStatus.  The domain object is
 * intentionally never released: it must outlive every session that uses it.
 */
#ifndef XMETAI_ONNX_PLUGINS_ORT_H_
#define XMETAI_ONNX_PLUGINS_ORT_H_

#include <onnxruntime_c_api.h>

#ifdef __cplusplus
extern "C" {
#endif

OrtStatus *ORT_API_CALL RegisterCustomOps(OrtSessionOptions *options, const OrtApiBase *api_base);

#ifdef __cplusplus
}
#endif

#endif /* XMETAI_ONNX_PLUGINS_ORT_H_ */

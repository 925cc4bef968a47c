/*
 * xmetai_recurrent.h — C ABI of the MI355X (gfx950) recurrent operators.
 *
 * Three operators of the ONNX domain "xmetai_plugins", with the reference's
 * input order, attribute names, defaults and validation:
 *
 *   SelectiveScanFn   (8 inputs)  reference: csrc/selective_scan/selective_scan_fn_ort.cpp:48-246
 *   Mamba3SisoFn      (11 inputs) reference: csrc/mamba3_siso/mamba3_siso_fn_ort.cpp:41-246
 *   GatedDeltaNet2Fn  (7 inputs)  reference: csrc/gated_deltanet2/gated_deltanet2_fn_ort.cpp:44-237
 *
 * The ONNX Runtime custom-op layer (RegisterCustomOps, declared in
 * xmetai_onnx_plugins_ort.h) unpacks OrtValues into xm_tensor_t descriptors,
 * reads node attributes into the attrs structs below and calls these entry
 * points with the ROCm EP compute stream and an allocator that forwards to
 * KernelContext_GetScratchBuffer.  A harness can call them directly with its
 * own device buffers and stream.
 *
 * Conventions
 *  - Every input is REQUIRED; an "optional" input is a tensor with zero
 *    elements (reference: ort_common.h:93-95).  Its data pointer may be NULL.
 *  - Tensors are dense, row-major, fp32 (elem_type == XM_ELEM_FLOAT), on the
 *    device that is current when the entry point is called.  The exceptions:
 *    cu_seqlens offsets are int64, and SelectiveScanFn's data tensors may be
 *    float16 or bfloat16 (its section says which).
 *  - Entry points return XM_OK or an xm_status_t error and, on error, write a
 *    NUL-terminated message into errbuf (when errbuf != NULL, errlen > 0).
 *    Messages match the reference's exception text where the reference has one.
 *  - *_forward never synchronises the host with the device, keeps no state
 *    between calls and is reentrant: concurrent calls on different streams
 *    are independent.  Work is enqueued on `stream` (a hipStream_t; NULL means
 *    the null stream).  Scratch comes from `alloc` in stream order; when
 *    `alloc` is NULL the library uses its own stream-ordered pool
 *    (hipMallocFromPoolAsync / hipFreeAsync on `stream`).
 *  - No host-visible side effects besides the output tensors.
 */
#ifndef XMETAI_RECURRENT_H_
#define XMETAI_RECURRENT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XM_MAX_RANK 8
#define XM_ELEM_FLOAT 1 /* ONNX TensorProto FLOAT */
#define XM_ELEM_INT64 7 /* ONNX TensorProto INT64 (cu_seqlens) */
#define XM_ELEM_FLOAT16 10  /* ONNX TensorProto FLOAT16 (SelectiveScanFn data) */
#define XM_ELEM_BFLOAT16 16 /* ONNX TensorProto BFLOAT16 (SelectiveScanFn data) */

typedef enum xm_status {
    XM_OK = 0,
    XM_ERR_INVALID_ARGUMENT = 1, /* shape, rank, dtype or attribute rejected */
    XM_ERR_UNSUPPORTED = 2,      /* a feature the operator does not support (v1 limits) */
    XM_ERR_DEVICE = 3,           /* a HIP runtime or launch error */
    XM_ERR_ALLOC = 4             /* the scratch allocator returned NULL */
} xm_status_t;

/* A borrowed device tensor. */
typedef struct xm_tensor {
    const void *data;              /* device pointer, may be NULL when a dim is 0 */
    int64_t shape[XM_MAX_RANK];
    int32_t rank;
    int32_t elem_type;             /* XM_ELEM_* (ONNX TensorProto values) */
} xm_tensor_t;

/* Stream-ordered scratch allocator.  alloc() must return memory that is
 * usable by work enqueued on the operator's stream after the call; free() may
 * be called right after the operator enqueues its last kernel (the memory is
 * reused only in stream order).  Reference: gated_deltanet2_fn_ort.cpp:89-111. */
typedef struct xm_allocator {
    void *ctx;
    void *(*alloc)(void *ctx, size_t bytes);
    void (*free)(void *ctx, void *ptr);
} xm_allocator_t;

/* ---- SelectiveScanFn ------------------------------------------------------
 * Inputs: 0 u [B,D,L]; 1 delta [B,D,L]; 2 A [D,N]; 3 B [D,N] | [B,N,L] |
 * [B,G,N,L]; 4 C (same forms); 5 D [D] or empty; 6 z [B,D,L] or empty;
 * 7 delta_bias [D] or empty.  Output 0: y [B,D,L], the un-gated scan output
 * (reference: selective_scan_fwd_kernel.cuh:272-281; z only feeds a discarded
 * buffer there, :283-301, so y never depends on z).
 * Element types: fp32 everywhere, or (a widening: the reference has half and
 * bfloat16 kernels, selective_scan_fwd_fp16.cu:9-10 and _bf16.cu, that its
 * fp32-only host, ort_common.h:90-92, cannot reach) u, delta, z and variable
 * B/C in XM_ELEM_FLOAT16 or XM_ELEM_BFLOAT16, one type for all of them, with
 * A, D, delta_bias and constant B/C in fp32: the reference's input_t /
 * weight_t split.  The arithmetic is fp32; y has u's element type and
 * last_state stays fp32.
 * Attributes (reference: selective_scan_fn_ort.cpp:50-56): delta_softplus
 * (int, default 0), return_last_state (int, default 0; the reference rejects
 * non-zero, here it selects the last-state output of
 * xm_selective_scan_forward_states).  */
typedef struct xm_selective_scan_attrs {
    int64_t delta_softplus;
    int64_t return_last_state;
} xm_selective_scan_attrs_t;

void xm_selective_scan_attrs_default(xm_selective_scan_attrs_t *attrs);
/* Session-time check of the attributes (reference: constructor, :50-56). */
int xm_selective_scan_check_attrs(const xm_selective_scan_attrs_t *attrs, char *errbuf, size_t errlen);
/* Run-time shape validation without touching the device (reference:
 * Compute, :58-117).  Writes the output shape and the scratch bytes the call
 * will request from the allocator. */
int xm_selective_scan_validate(const xm_tensor_t *inputs, size_t n_inputs,
                               const xm_selective_scan_attrs_t *attrs, int64_t *out_shape,
                               int32_t *out_rank, size_t *scratch_bytes, char *errbuf, size_t errlen);
/* Validate and enqueue.  `out` is a device buffer of prod(out_shape) elements
 * of u's type.  With return_last_state != 0 this entry point fails (use the
 * one below). */
int xm_selective_scan_forward(const xm_tensor_t *inputs, size_t n_inputs,
                              const xm_selective_scan_attrs_t *attrs, void *out, void *stream,
                              const xm_allocator_t *alloc, char *errbuf, size_t errlen);
/* As above; with return_last_state != 0 it also writes the scan state after
 * the last token to `last_state`, a device buffer [B, D, N] (zeros when L = 0).
 * The reference rejects return_last_state != 0 (selective_scan_fn_ort.cpp:52-55);
 * this is a widening with no counterpart there: the state is the `last_state`
 * of the Mamba selective_scan_fn interface.  `last_state` is ignored (may be
 * NULL) when return_last_state == 0. */
int xm_selective_scan_forward_states(const xm_tensor_t *inputs, size_t n_inputs,
                                     const xm_selective_scan_attrs_t *attrs, void *out, float *last_state,
                                     void *stream, const xm_allocator_t *alloc, char *errbuf,
                                     size_t errlen);

/* ---- Mamba3SisoFn ---------------------------------------------------------
 * Inputs: 0 Q [B,T,Hq,N]; 1 K [B,T,Hq,N]; 2 V [B,T,H,P]; 3 ADT [B,H,T];
 * 4 DT [B,H,T]; 5 Trap [B,H,T]; 6 Q_bias [H,N]; 7 K_bias [H,N];
 * 8 Angles [B,T,H,A]; 9 D [H] or empty; 10 Z [B,T,H,P] or empty.
 * Output 0: [B,T,H,P] (reference: mamba3_siso_fn_ort.cpp:61-111).
 * Attributes (reference: :43-59): chunk_size (default 64, must be > 0, not
 * otherwise used), has_d and has_z (default 1, must match the presence of D
 * and Z), return_final_states and has_input_states (default 0; the reference
 * rejects non-zero, here they select the states below), has_cu_seqlens
 * (default 0; the reference rejects non-zero, here it selects packed
 * sequences, below).
 * States (a widening with no counterpart in the reference, which rejects them
 * at mamba3_siso_fn_ort.cpp:50-55): ssm [B,H,P,N], angle [B,H,A], k [B,H,N],
 * v [B,H,P] -- the scan state and the angle state after the last token, that
 * token's rotated k and its V.  With has_input_states != 0 they are inputs
 * 11-14 (15 inputs) and the scan starts from ssm + v (x) k * DT_0 *
 * (1 - sigmoid(Trap_0)) and angle, so that two calls chained through the
 * states give the outputs and states of one call.
 * Packed sequences (a widening; the reference rejects has_cu_seqlens at
 * mamba3_siso_fn_ort.cpp:56-58): 16 inputs, input 15 cu_seqlens, int64
 * (XM_ELEM_INT64) [N+1], the token offsets of N sequences packed along T
 * (inputs 11-14 empty unless has_input_states != 0); the tensors have batch 1
 * and the states are [N,H,...], one per sequence.  Offsets are read on the
 * device: each is clamped into [0, T], a sequence ending before it starts is
 * empty and passes its states through.  */
typedef struct xm_mamba3_siso_attrs {
    int64_t chunk_size;
    int64_t has_d;
    int64_t has_z;
    int64_t return_final_states;
    int64_t has_input_states;
    int64_t has_cu_seqlens;
} xm_mamba3_siso_attrs_t;

void xm_mamba3_siso_attrs_default(xm_mamba3_siso_attrs_t *attrs);
int xm_mamba3_siso_check_attrs(const xm_mamba3_siso_attrs_t *attrs, char *errbuf, size_t errlen);
int xm_mamba3_siso_validate(const xm_tensor_t *inputs, size_t n_inputs,
                            const xm_mamba3_siso_attrs_t *attrs, int64_t *out_shape,
                            int32_t *out_rank, size_t *scratch_bytes, char *errbuf, size_t errlen);
/* With return_final_states != 0 this entry point fails (use the one below). */
int xm_mamba3_siso_forward(const xm_tensor_t *inputs, size_t n_inputs,
                           const xm_mamba3_siso_attrs_t *attrs, float *out, void *stream,
                           const xm_allocator_t *alloc, char *errbuf, size_t errlen);
/* As above; with return_final_states != 0 it also writes the four states
 * after the last token to device buffers ssm_state [B,H,P,N], angle_state
 * [B,H,A], k_state [B,H,N] and v_state [B,H,P] (the layouts inputs 11-14
 * take).  The buffers are ignored (may be NULL) when return_final_states == 0.
 * A widening with no counterpart in the reference (mamba3_siso_fn_ort.cpp:50-52). */
int xm_mamba3_siso_forward_states(const xm_tensor_t *inputs, size_t n_inputs,
                                  const xm_mamba3_siso_attrs_t *attrs, float *out, float *ssm_state,
                                  float *angle_state, float *k_state, float *v_state, void *stream,
                                  const xm_allocator_t *alloc, char *errbuf, size_t errlen);

/* ---- GatedDeltaNet2Fn -----------------------------------------------------
 * Inputs: 0 q [B,T,H,K]; 1 k [B,T,H,K]; 2 v [B,T,H,V]; 3 g [B,T,H,K]
 * (log decay, per key); 4 beta [B,T,H,K]; 5 w [B,T,H,V] (write gate);
 * 6 initial_state [B,H,K,V] or empty.  Output 0: [B,T,H,V]
 * (reference: gated_deltanet2_fn_ort.cpp:66-142, :187-219).
 * Attributes (reference: :46-64): scale (float, default 1.0, positive and
 * finite), use_qk_l2norm_in_kernel (default 1), output_final_state (default
 * 0; the reference rejects non-zero, here it selects the final-state output
 * of xm_gated_deltanet2_forward_states), has_cu_seqlens (default 0; the
 * reference rejects non-zero, here it selects packed sequences, below),
 * use_gate_in_kernel, state_v_first (default 0; non-zero rejected).
 * Packed sequences (a widening with no counterpart in the reference, which
 * rejects has_cu_seqlens at gated_deltanet2_fn_ort.cpp:55-57): with
 * has_cu_seqlens != 0 input 7 is cu_seqlens, int64 (XM_ELEM_INT64) [N+1], the
 * token offsets of N sequences packed along T; q..w are [1,T,H,.] and
 * initial_state / final_state are [N,H,K,V], one state per sequence.  Offsets
 * are read on the device: they should rise from 0 to T; each one is clamped
 * into [0, T] and a sequence ending before it starts is empty (its state
 * passes through).  head_k up to 512.  */
typedef struct xm_gated_deltanet2_attrs {
    float scale;
    int64_t use_qk_l2norm_in_kernel;
    int64_t output_final_state;
    int64_t use_gate_in_kernel;
    int64_t has_cu_seqlens;
    int64_t state_v_first;
} xm_gated_deltanet2_attrs_t;

void xm_gated_deltanet2_attrs_default(xm_gated_deltanet2_attrs_t *attrs);
int xm_gated_deltanet2_check_attrs(const xm_gated_deltanet2_attrs_t *attrs, char *errbuf, size_t errlen);
int xm_gated_deltanet2_validate(const xm_tensor_t *inputs, size_t n_inputs,
                                const xm_gated_deltanet2_attrs_t *attrs, int64_t *out_shape,
                                int32_t *out_rank, size_t *scratch_bytes, char *errbuf,
                                size_t errlen);
int xm_gated_deltanet2_forward(const xm_tensor_t *inputs, size_t n_inputs,
                               const xm_gated_deltanet2_attrs_t *attrs, float *out, void *stream,
                               const xm_allocator_t *alloc, char *errbuf, size_t errlen);
/* As above; with output_final_state != 0 it also writes the state after the
 * last token to `final_state`, a device buffer [B, H, K, V] (initial_state's
 * layout, so a later call can continue from it).  A widening with no
 * counterpart in the reference, which rejects output_final_state != 0
 * (gated_deltanet2_fn_ort.cpp:49-51).  `final_state` is ignored (may be NULL)
 * when output_final_state == 0. */
int xm_gated_deltanet2_forward_states(const xm_tensor_t *inputs, size_t n_inputs,
                                      const xm_gated_deltanet2_attrs_t *attrs, float *out,
                                      float *final_state, void *stream, const xm_allocator_t *alloc,
                                      char *errbuf, size_t errlen);

/* xm_gated_deltanet2_forward with no allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * scratch comes from a fixed 64 MiB array in device memory that each GPU the
 * library runs on holds until the process ends; the chunked path's windows
 * and the preparation chunks of head_k > 512 shrink to fit it, and a call that
 * cannot fit (e.g. a carried state of 64 MiB or more) fails with
 * XM_ERR_UNSUPPORTED before anything is enqueued.  It calls no hipMalloc or
 * hipFree.  Every call on a GPU shares that GPU's array: calls that overlap on
 * one GPU (concurrent streams) race and must be serialised by the caller.
 * Results equal xm_gated_deltanet2_forward's, except where that call splits
 * the sequence into concurrently run segments (few heads, 32+ chunks) with
 * more scratch than the array holds: this entry point then steps the
 * sequence in windows, and the two agree within the fp32 tolerance of two
 * evaluation orders.  output_final_state must be 0. */
int xm_gated_deltanet2_forward_noalloc(const xm_tensor_t *inputs, size_t n_inputs,
                                       const xm_gated_deltanet2_attrs_t *attrs, float *out, void *stream,
                                       char *errbuf, size_t errlen);

/* ---- SoftmaxCPU (CPU execution provider) ------------------------------------
 * Softmax of a HOST fp32 tensor of any rank along `axis` (ONNX attribute
 * "axis", int, default -1; negative values count from the last dimension).
 * Per line: subtract the maximum, exp, sum in axis order, multiply by
 * (sum > 0 ? 1/sum : 0).  An empty tensor returns XM_OK without checking the
 * axis; otherwise an axis outside [-rank, rank) fails with "SoftmaxCPU axis
 * out of range".  `out` has the input's shape and may not alias `in`.
 * Reference: csrc/softmax_cpu/softmax_cpu_ort.cpp:20-114 (kernel), :79-88
 * (axis attribute). */
int xm_softmax_cpu(const float *in, const int64_t *shape, int32_t rank, int64_t axis, float *out,
                   char *errbuf, size_t errlen);

/* ---- Kernel-selection overrides (tests and tuning) ---------------------------
 * Process-wide switches that force a kernel variant the dispatchers would not
 * pick by themselves, so that parity tests can run every variant; value 0
 * restores the dispatcher's own choice.  Production callers never need them.
 *   "gdn2_path"      1: GatedDeltaNet2Fn sequential fused kernel (headdim_k <= 512)
 *   "gdn2_pairwise"  1: every chunk of the chunked GDN-2 path forms A and M pairwise
 *   "gdn2_rows"      1, 2, 4: rows of 16 lanes per value column of the fused kernel
 *   "m3_path"        1: Mamba3SisoFn token-by-token kernel
 *   "ss_lpc"         1, 2, 4, 8, 16: SelectiveScanFn lanes per channel (d_state <= 16)
 *   "ss_split"       1: SelectiveScanFn channel-block kernel only; 2: the
 *                    sequence-split kernel wherever it applies
 *   "gdn2_kpw4"      1: chunked GDN-2 above 128 keys with 4 key tiles per wave
 *   "gdn2_windowed"  1: chunked GDN-2 in windows of 128 chunks
 *   "gdn2_split"     1: chunked GDN-2 never split along the sequence; 2: split
 *                    into up to four segments wherever the sequence has 2+ chunks;
 *                    3: two unequal segments, the second two column tiles per
 *                    workgroup (where such a kernel is built, 2+ chunks)
 *   "gdn2_ct"        1, 2: value-column tiles (of 16 columns) per chunked GDN-2
 *                    recurrence workgroup, 2 where such a kernel is built (by
 *                    default 2 where one tile per workgroup would launch more
 *                    workgroups than the device has CUs)
 * The values are read with one atomic load per launch; a change affects calls
 * made after it.  No counterpart in the reference (its variants are fixed at
 * compile time).  xm_set_kernel_override returns XM_ERR_INVALID_ARGUMENT for
 * an unknown name or value; xm_get_kernel_override returns -1 for an unknown
 * name. */
int xm_set_kernel_override(const char *name, int64_t value, char *errbuf, size_t errlen);
int64_t xm_get_kernel_override(const char *name);

/* ---- Library ---------------------------------------------------------------
 * Version string and a description of the build (target, kernel variants). */
const char *xm_version(void);
/* The kernels the calling host thread's last *_forward / *_forward_states
 * call enqueued, in launch order, ';'-separated, each with its template
 * arguments and " xN" when launched N > 1 times, e.g.
 * "Gdn2ChunkPrepKernel x2;Gdn2ChunkRecurKernel<2,4> x2" (booleans as 0/1;
 * rocprofv3 prints the same kernels as demangled signatures).  Diagnostics
 * for benchmarks and tests; the string is valid until the thread's next call.
 * No counterpart in the reference. */
const char *xm_last_launches(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* XMETAI_RECURRENT_H_ */

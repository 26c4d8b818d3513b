/*
 * accel_hip: the C-ABI device layer behind AccelEP's accel::Device seam, on one
 * MI355X (gfx950). Plain pointers and sizes only; every compute call is a HIP
 * kernel launched on the library's single stream.
 *
 * Each entry point replaces one call of the reference's device contract
 * (AccelEP include/accel/device.h, include/accel/runtime.h) and keeps its
 * argument meaning and error behaviour: where the reference throws, the call
 * returns the status code named for that exception type and leaves a message in
 * accel_hip_last_error(). The C++ shim (include/accel/device.h,
 * accel::CreateHipDevice) rethrows the same exception types.
 *
 * Memory: every pointer argument named as a device pointer must come from
 * accel_hip_allocate (or be an offset into such an allocation). Calls are
 * stream-ordered; accel_hip_copy_d2h and accel_hip_peek return after the data
 * is on the host.
 */
#ifndef ACCEL_HIP_H_
#define ACCEL_HIP_H_

#include <stddef.h>
#include <stdint.h>

#define ACCEL_HIP_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: the exception the reference throws for the same condition. */
enum {
  ACCEL_HIP_OK = 0,
  ACCEL_HIP_INVALID_ARGUMENT = 1, /* std::invalid_argument */
  ACCEL_HIP_OVERFLOW = 2,         /* std::overflow_error */
  ACCEL_HIP_LOGIC_ERROR = 3,      /* std::logic_error */
  ACCEL_HIP_BAD_ALLOC = 4,        /* std::bad_alloc */
  ACCEL_HIP_RUNTIME_ERROR = 5     /* a HIP runtime failure (no reference counterpart) */
};

enum { ACCEL_HIP_ACT_NONE = 0, ACCEL_HIP_ACT_RELU = 1, ACCEL_HIP_ACT_GELU = 2 }; /* accel::Activation */

/* accel::DeviceBuffer (include/accel/device.h:28-32). id 0 marks a slice. */
typedef struct AccelHipBuffer {
  void* data;
  size_t bytes;
  uint64_t id;
} AccelHipBuffer;

/* accel::QuantPlane (include/accel/runtime.h:71-78) with the shape inline.
 * q/scale/zero are device pointers; zero is NULL when the op has none. */
typedef struct AccelHipQuantPlane {
  const int8_t* q;
  const float* scale;
  const int8_t* zero;
  int32_t rank; /* 1..8 */
  int64_t shape[8];
  int64_t axis; /* < 0: one scale (and zero) for the whole tensor */
  int64_t offset;
} AccelHipQuantPlane;

/* accel::AcceleratorStats (include/accel/runtime.h:11-21). */
typedef struct AccelHipStats {
  int64_t matmul_ops, gemm_ops, kernel_matmuls, relu_epilogues, gelu_epilogues, add_epilogues, device_transposes,
      bytes_to_device, bytes_to_host;
} AccelHipStats;

/* Fused register epilogue applied to C before it is stored (no reference
 * counterpart as one call: it is the reference's call sequence
 * MatMul/MatMulQuantized -> GemmEpilogue(alpha, bias, beta, act) ->
 * GemmEpilogue(residual) (src/runtime.cc:332-344,709-719) -> RmsNorm
 * (src/ep.cc:1602-1626), with the same rounding steps:
 *   v = alpha*acc; if bias: v = v + beta*bias[bcast(i, j)]; act(v);
 *   if residual: v = v + residual[i*n + j]; store v;
 *   if rms_weight: rms_out[i, :] = RmsNorm(v[i, :]) with eps = rms_eps. */
typedef struct AccelHipEpilogue {
  float alpha;
  float beta;
  const float* bias; /* device pointer or NULL */
  int32_t bias_rank; /* 0..2, right-aligned against [m, n] */
  int64_t bias_shape[2];
  int32_t activation;    /* ACCEL_HIP_ACT_* */
  const float* residual; /* device pointer [m, n] or NULL */
  const float* rms_weight; /* device pointer [n] or NULL */
  float rms_eps;
  float* rms_out; /* device pointer [m, n]; required when rms_weight is set */
} AccelHipEpilogue;

/* ---- runtime ----------------------------------------------------------------------------- */
/* Message of this thread's last failed call; "" after a call that worked. */
ACCEL_HIP_API const char* accel_hip_last_error(void);
/* Binds GPU 0 and creates the stream. Every other entry point calls it on first use. */
ACCEL_HIP_API int accel_hip_init(void);
/* Waits for all work on the library's stream. */
ACCEL_HIP_API int accel_hip_synchronize(void);
/* gcnArchName of the bound GPU, e.g. "gfx950:sramecc+:xnack-". */
ACCEL_HIP_API const char* accel_hip_device_arch(void);

/* ---- heap and copies: Device::Allocate/Free/CopyHostToDevice/CopyDeviceToHost ----------
 * (include/accel/device.h:75-79; semantics src/sim_device.cc:133-183). Allocate zero-fills,
 * returns a non-null pointer for 0 bytes, and mints a process-wide id from 1. Free of a null
 * pointer is a no-op; an unknown (data, bytes, id) triple is ACCEL_HIP_LOGIC_ERROR. Copies of
 * 0 bytes do nothing; a null pointer or bytes > buffer.bytes is ACCEL_HIP_INVALID_ARGUMENT;
 * each copy adds to bytes_to_device / bytes_to_host. */
ACCEL_HIP_API int accel_hip_allocate(size_t bytes, AccelHipBuffer* out);
ACCEL_HIP_API int accel_hip_free(AccelHipBuffer buffer);
ACCEL_HIP_API int accel_hip_copy_h2d(AccelHipBuffer dst, const void* src, size_t bytes);
ACCEL_HIP_API int accel_hip_copy_d2h(void* dst, AccelHipBuffer src, size_t bytes);
/* Uncounted reads/writes: the reference's host code reads device memory through raw
 * pointers without a counted copy (src/llama_model.cc:118,146,172,204). */
ACCEL_HIP_API int accel_hip_peek(void* dst, const void* device_src, size_t bytes);
ACCEL_HIP_API int accel_hip_poke(void* device_dst, const void* src, size_t bytes);
/* LiveDeviceAllocs (include/accel/device.h:133-135). */
ACCEL_HIP_API int64_t accel_hip_live_allocs(void);
/* Releases cached device blocks back to HIP (does not change live counts). */
ACCEL_HIP_API int accel_hip_trim(void);

/* ---- stats (src/runtime.cc:420-458) and packed-GEMM probes (src/sim_device.cc:379-385) --- */
ACCEL_HIP_API void accel_hip_get_stats(AccelHipStats* out);
ACCEL_HIP_API void accel_hip_reset_stats(void);
ACCEL_HIP_API int64_t accel_hip_packed_matmul_calls(void);
ACCEL_HIP_API int64_t accel_hip_packed_k_trips(void);
ACCEL_HIP_API void accel_hip_reset_packed_probes(void);

/* ---- compute ---------------------------------------------------------------------------- */
/* Device::MatMul (include/accel/device.h:81-82; src/sim_device.cc:185-196): row-major
 * C[m, n] = A[m, k] @ B[k, n], overwrites C (zeros when k == 0). fp32 MFMA. */
ACCEL_HIP_API int accel_hip_matmul(AccelHipBuffer a, AccelHipBuffer b, AccelHipBuffer c, int64_t m, int64_t k,
                                   int64_t n);
/* accel::MatMulQuantized (include/accel/runtime.h:124-125; src/sim_device.cc:541-602).
 * Device pointers; a NULL plane reads the float pointer. Either side may be quantized.
 * w = (float(q) - float(zero)) * scale at the plane's coordinate. m <= 16: the int8 GEMV
 * (VALU for m <= 2, exact bf16-split products on the matrix cores for 3 <= m <= 16). Above
 * that, an int8 weight with per-column or whole-tensor scale, no zero points and k % 32 == 0
 * runs on the bf16 matrix cores with the activation split exactly into three bf16 parts (the
 * weight staged once as bf16); other planes on the fp32 MFMA GEMM with the int8 panel
 * dequantized in LDS. */
ACCEL_HIP_API int accel_hip_matmul_quantized(const float* a, const AccelHipQuantPlane* a_quant, const float* b,
                                             const AccelHipQuantPlane* b_quant, float* c, int64_t m, int64_t k,
                                             int64_t n);
/* Weight preparation. No counterpart in the reference, whose MatMulQuantized dequantizes each
 * panel on the fly (src/sim_device.cc:541-602); it belongs where the reference uploads and
 * binds the weight (UploadDequantized and BindConstant, src/ep.cc:843-900,1430-1463). Builds
 * now, on the library stream, the staged copies of the int8 weight b_quant ([k, n] at its
 * offset) that the matmuls otherwise build at the weight's first use: layouts is a mask of
 * ACCEL_HIP_STAGE_*, 0 for every layout this plane's form allows. A copy lasts until the
 * weight's allocation is freed or written. Refused (ACCEL_HIP_RUNTIME_ERROR) during a graph
 * capture; ACCEL_HIP_INVALID_ARGUMENT for a layout the plane cannot take or a weight outside
 * this library's heap. *staged (if not NULL) receives the layouts built. */
#define ACCEL_HIP_STAGE_GEMV_TILES 1u  /* 8-column tiles: the int8 GEMV at m <= 4 where groups are not taken */
#define ACCEL_HIP_STAGE_GEMV_GROUPS 2u /* group-interleaved tiles: the bf16-split GEMV, 3 <= m <= 16 */
#define ACCEL_HIP_STAGE_GEMM_BF16 4u   /* bf16 in MFMA operand order: the int8-weight GEMM, m > 16 */
#define ACCEL_HIP_STAGE_GEMM_SMALL 8u  /* bf16 in the small GEMM's operand order: m > 16, k <= 768 */
#define ACCEL_HIP_STAGE_ALL 15u
ACCEL_HIP_API int accel_hip_prepare_quantized(const AccelHipQuantPlane* b_quant, int64_t k, int64_t n,
                                              uint32_t layouts, uint32_t* staged);
/* Exact products (no reference counterpart as a switch; it selects the reference's own
 * arithmetic). When on, every matmul entry point sums each output in k order from zero with
 * each product rounded before its add, and dequantizes an int8 operand per element as
 * (float(q) - float(zero)) * scale: the bits of ReferenceMatMul / MatMulQuantized
 * (src/sim_device.cc:387-402,541-602). When off (the default) the GEMMs and GEMVs add in
 * their own order: within 2*gamma_K*(|A|@|B|) of the exact product. Process-wide;
 * accel_hip_exact_products() reads the setting (1 on, 0 off). */
ACCEL_HIP_API int accel_hip_set_exact_products(int32_t on);
ACCEL_HIP_API int32_t accel_hip_exact_products(void);
/* Fused forms of the two calls above (see AccelHipEpilogue). Count as one kernel matmul
 * each, like the unfused call; the caller notes its epilogue counters as the runtime does. */
ACCEL_HIP_API int accel_hip_matmul_fused(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n,
                                         const AccelHipEpilogue* epilogue);
ACCEL_HIP_API int accel_hip_matmul_quantized_fused(const float* a, const AccelHipQuantPlane* a_quant, const float* b,
                                                   const AccelHipQuantPlane* b_quant, float* c, int64_t m, int64_t k,
                                                   int64_t n, const AccelHipEpilogue* epilogue);
/* No counterpart in the reference. accel_hip_matmul_quantized_fused for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same arguments, checks, results and counters. It calls no hipMalloc,
 * hipFree or other allocating routine: the scratch its kernels need (split-K partial sums,
 * arrival counters, a dequantized operand for plane layouts the kernels do not index) comes
 * from one fixed 64 MiB device array per GPU, held until the process ends, and a call whose
 * scratch would exceed it returns ACCEL_HIP_INVALID_ARGUMENT. A staged GEMV copy of W is read
 * only if an earlier call built one (otherwise W is read in place). Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU race. */
ACCEL_HIP_API int accel_hip_matmul_quantized_fused_noalloc(const float* a, const AccelHipQuantPlane* a_quant,
                                                           const float* b, const AccelHipQuantPlane* b_quant, float* c,
                                                           int64_t m, int64_t k, int64_t n,
                                                           const AccelHipEpilogue* epilogue);
/* Device::Transpose (device.h:84-85; src/sim_device.cc:198-209): dst[j, i] = src[i, j]. */
ACCEL_HIP_API int accel_hip_transpose(AccelHipBuffer src, AccelHipBuffer dst, int64_t rows, int64_t cols);
/* Device::GemmEpilogue (device.h:87-92; src/sim_device.cc:211-245). bias may be NULL. */
ACCEL_HIP_API int accel_hip_gemm_epilogue(AccelHipBuffer c, int64_t m, int64_t n, float alpha,
                                          const AccelHipBuffer* bias, int32_t bias_rank, const int64_t* bias_shape,
                                          float beta, int32_t activation);
/* Device::Embedding (device.h:94-96; src/sim_embed.cc:9-20). An id outside [0, vocab) is
 * ACCEL_HIP_INVALID_ARGUMENT ("token id is outside the vocabulary"), detected on the device. */
ACCEL_HIP_API int accel_hip_embedding(AccelHipBuffer ids, int64_t id_offset, AccelHipBuffer table, AccelHipBuffer out,
                                      int64_t seq, int64_t hidden, int64_t vocab);
/* Embedding from an int8 table with one scale per row: out = float(q) * scale[id], the
 * same fl(q*s) value a float table quantized that way holds. No reference counterpart as
 * one call; used by the int8 Llama. */
ACCEL_HIP_API int accel_hip_embedding_q8(AccelHipBuffer ids, int64_t id_offset, const int8_t* table,
                                         const float* row_scale, AccelHipBuffer out, int64_t seq, int64_t hidden,
                                         int64_t vocab);
/* Device::RmsNorm (device.h:98-100; src/sim_rmsnorm.cc:7-20). */
ACCEL_HIP_API int accel_hip_rms_norm(AccelHipBuffer x, AccelHipBuffer weight, AccelHipBuffer y, int64_t rows,
                                     int64_t dim, float eps, int64_t row_offset);
/* Device::Rope (device.h:102-104; src/sim_rope.cc:5-21). */
ACCEL_HIP_API int accel_hip_rope(AccelHipBuffer states, AccelHipBuffer cos_table, AccelHipBuffer sin_table,
                                 int64_t seq, int64_t n_heads, int64_t head_dim, int64_t position);
/* Device::AppendCache (device.h:106-108; src/sim_cache.cc:8-13). */
ACCEL_HIP_API int accel_hip_append_cache(AccelHipBuffer src, AccelHipBuffer cache, int64_t seq, int64_t position,
                                         int64_t n_heads, int64_t head_dim);
/* Device::Attention (device.h:110-112; src/sim_attend.cc:9-46). scores is not used as
 * scratch by the HIP kernel but must still be large enough, as in the reference. */
ACCEL_HIP_API int accel_hip_attention(AccelHipBuffer q, AccelHipBuffer k, AccelHipBuffer v, AccelHipBuffer scores,
                                      AccelHipBuffer out, int64_t seq, int64_t position, int64_t heads,
                                      int64_t kv_heads, int64_t head_dim);
/* Device::SiluMul (device.h:114-115; src/sim_silu.cc:8-13). */
ACCEL_HIP_API int accel_hip_silu_mul(AccelHipBuffer gate, AccelHipBuffer up, int64_t count);
/* Device::ResidualAdd (device.h:117-118; src/sim_add.cc:5-9). */
ACCEL_HIP_API int accel_hip_residual_add(AccelHipBuffer dest, AccelHipBuffer extra, int64_t count);
/* Device::SampleToken (device.h:120-124; src/sim_sample.cc:25-115). *rng_state is read
 * before and written after the draw, as the reference's xorshift32 state. */
ACCEL_HIP_API int accel_hip_sample_token(AccelHipBuffer logits, AccelHipBuffer chosen_ids, int64_t chosen_index,
                                         int64_t vocab, float temperature, uint32_t* rng_state, int32_t top_k);

/* ---- timing ----------------------------------------------------------------------------- */
/* Milliseconds between two HIP events recorded on the library's stream around `iters`
 * back-to-back calls of fn(user); returns < 0 on failure. Used by bench.py. */
typedef int (*AccelHipWorkFn)(void* user);
ACCEL_HIP_API double accel_hip_time_ms(AccelHipWorkFn fn, void* user, int32_t iters);
/* Records/reads events on the library's stream (for timing regions driven from Python), in
 * slots 0 .. 15. Recorded during a capture (accel_hip_capture_begin), the event becomes a node
 * of the graph, recorded each time the graph is replayed, and stays timeable. */
ACCEL_HIP_API int accel_hip_event_record(int32_t slot);
ACCEL_HIP_API double accel_hip_event_elapsed_ms(int32_t start_slot, int32_t end_slot);

/* ---- HIP graphs --------------------------------------------------------------------------
 * Captures the kernels that the calls between begin and end enqueue on the library stream
 * into an executable graph, replayed by accel_hip_graph_launch. Calls made during a capture
 * must not synchronize (no counted copies, allocations or first-use workspace growth):
 * warm them up once before capturing. No reference counterpart (the reference runs on the
 * host); used to replay a fixed launch sequence without host launch overhead. */
ACCEL_HIP_API int accel_hip_capture_begin(void);
ACCEL_HIP_API int accel_hip_capture_end(void** graph_exec);
ACCEL_HIP_API int accel_hip_graph_launch(void* graph_exec, int32_t times);
ACCEL_HIP_API int accel_hip_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif

#endif /* ACCEL_HIP_H_ */

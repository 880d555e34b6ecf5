/*
 * qmm.h -- C ABI of the MI355X (gfx950) quantized-matmul backend.
 *
 * This is the drop-in boundary for Candle's quantized matmul path as the
 * reference LLM engine uses it:
 *   QuantizedLinear::{quantize, forward}  crates/llm/candle-llm/src/primitives/quant.rs:26-43
 *   QTensor::quantize / QMatMul::from_qtensor / QMatMul::forward (candle-core @1e6aa85e,
 *     called at quant.rs:27, :29, :38)
 *   QTensor::new(QStorage::from_data(..)) crates/media/candle-gen/candle-gen/src/quant/repack.rs:202-203
 *   QTensor::dequantize                   crates/llm/candle-llm/src/gguf.rs:104
 * and for the kernel-level launchers those calls reach on a GPU:
 *   launch_mmvq_gguf_quantize_q8_1_f32    crates/media/candle-gen/vendor/candle-kernels/src/ffi.rs:412-419
 *   launch_mmvq_gguf_{q8_0,q4_k,q6_k}_f32_plain  ffi.rs:217-227, 250-260, 272-282
 *   launch_mmq_gguf_{q4_k,q6_k}           ffi.rs:583-598, 615-630
 *   moe_gemm_gguf                         ffi.rs:25-39
 *
 * Conventions (deliberately stricter than the reference's void launchers):
 *   - every entry point returns an int status (QMM_OK == 0); qmm_last_error()
 *     gives a message for the calling thread;
 *   - all tensors are device pointers owned by the caller unless a function
 *     says otherwise; `stream` is a hipStream_t (NULL = the default stream);
 *   - weights live in opaque qmm_qtensor handles created from GGML block bytes
 *     or by quantizing f32 on the device; the handle owns its device memory;
 *   - a kernel image that cannot be loaded for the current device is an error
 *     (QMM_ERR_NO_KERNEL), never a silent no-op.
 * Kernels are launched only with hipModuleLaunchKernel from a gfx950 code
 * object embedded in the library.
 */
#ifndef QMM_H
#define QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
    QMM_OK = 0,
    QMM_ERR_INVALID = 1,     /* bad argument: shape, dtype, null pointer, size   */
    QMM_ERR_HIP = 2,         /* a HIP runtime call failed                         */
    QMM_ERR_NO_KERNEL = 3,   /* code object or kernel missing for this device     */
    QMM_ERR_UNSUPPORTED = 4, /* valid request this build does not implement       */
    QMM_ERR_OOM = 5          /* device allocation failed                          */
};

/* GGML dtype tags (GGUF numbering, crates/llm/mlx-llm/src/gguf/dequant.rs:87-113). */
enum {
    QMM_F32 = 0,
    QMM_F16 = 1,   /* dense outputs of qmm_qtensor_dequantize_to */
    QMM_BF16 = 30,
    QMM_Q8_0 = 8,  /* 34 B / 32:   f16 d, i8 qs[32]                          */
    QMM_Q4K = 12,  /* 144 B / 256: f16 d, f16 dmin, u8 scales[12], u8 qs[128] */
    QMM_Q6K = 14,  /* 210 B / 256: u8 ql[128], u8 qh[64], i8 scales[16], f16 d */
    QMM_Q8K = 15   /* 292 B / 256: f32 d, i8 qs[256], i16 bsums[16] (activations only) */
};

typedef struct qmm_qtensor qmm_qtensor;

/* Last error message of the calling thread ("" if none). */
const char *qmm_last_error(void);

/* Load the kernel code object on `device` (optional: every entry point loads it
 * lazily for the current device). */
int qmm_init(int device);

/* Re-read the QMM_* tuning overrides from the environment (kernel and launch
 * shape choices for sweeps and tests). They are read once, at the first call,
 * and then only here: a launch never consults the environment. No counterpart
 * in the reference (its launchers take no overrides). */
void qmm_reload_tuning(void);

/* GGML geometry: elements per block, bytes per block, and the activation type a
 * weight type multiplies against (Q8_0 -> Q8_0, Q4K/Q6K -> Q8K). -1 if unknown.
 * (GgmlDType::block_size / type_size / vec_dot_type.) */
int qmm_block_size(int dtype);
int qmm_type_size(int dtype);
int qmm_vec_dot_type(int dtype);

/* QTensor::new(QStorage::from_data(bytes, device, dtype), (n, k)).
 * `bytes` holds n*k/block_size GGML blocks, row-major over n then k, on the
 * host (bytes_on_device = 0) or on the current device (= 1). The bytes are
 * copied into the handle's own device layout; the caller keeps `bytes`. */
int qmm_qtensor_from_ggml(int dtype, int64_t n, int64_t k, const void *bytes, int bytes_on_device,
                          void *stream, qmm_qtensor **out);

/* QTensor::quantize(&Tensor f32 [n, k], dtype) computed on the device:
 * `w` is a device pointer to n*k f32 (row-major). The result's GGML bytes
 * equal those of candle's CPU from_float for the same input. */
int qmm_qtensor_quantize(int dtype, int64_t n, int64_t k, const float *w, void *stream,
                         qmm_qtensor **out);

/* QTensor::dequantize: n*k f32 into the device buffer `dst`. */
int qmm_qtensor_dequantize(const qmm_qtensor *t, float *dst, void *stream);

/* qmm_qtensor_dequantize to a dense [n, k] of out_dtype QMM_F32, QMM_F16 or
 * QMM_BF16 (each value rounded to nearest even from its f32 dequantization):
 * candle's QTensor::dequantize_f16 and the dequant-dense matmul strategy's
 * weight.dequantize(device).to_dtype(x.dtype) (candle-gen/src/quant/mod.rs:
 * 515-533; QMatMul::forward_via_f16 at candle-gen-lens/src/text_encoder.rs:
 * 518-529). */
int qmm_qtensor_dequantize_to(const qmm_qtensor *t, void *dst, int out_dtype, void *stream);

/* Export the tensor as GGML block bytes (qmm_qtensor_ggml_bytes() of them) into
 * `dst` on the host (dst_on_device = 0, synchronous) or the device (= 1). */
int qmm_qtensor_to_ggml(const qmm_qtensor *t, void *dst, int dst_on_device, void *stream);

/* Shape and dtype; size of the GGML byte image. */
int qmm_qtensor_info(const qmm_qtensor *t, int *dtype, int64_t *n, int64_t *k);
size_t qmm_qtensor_ggml_bytes(const qmm_qtensor *t);

/* Free a handle and its device memory (NULL is ignored). */
void qmm_qtensor_free(qmm_qtensor *t);

/* VecDotType::from_float on the device (replaces launch_mmvq_gguf_quantize_q8_1_f32,
 * ffi.rs:412-419): x is f32 [m, k] with row stride ldx (elements); xq receives
 * m rows of k/block_size blocks of `vdtype` (QMM_Q8_0 or QMM_Q8K), GGML bytes,
 * contiguous. Bytes equal the CPU quantizer's for the same input. */
int qmm_quantize_rows(int vdtype, const float *x, int64_t m, int64_t k, int64_t ldx, void *xq,
                      void *stream);

/* Bytes of workspace qmm_matmul needs for m activation rows (for m > 8: the
 * GEMM's quantized activation planes plus, when the weight's output tiles
 * cover fewer than half the CUs, f32 split-K partials). */
size_t qmm_matmul_workspace_size(const qmm_qtensor *w, int64_t m);

/* QMatMul::forward: y[i, j] = sum_k x[i, k] * W[j, k] for i < m, j < n, with x
 * quantized to W's vec-dot type first (as Candle's CPU path does).
 * x: f32 [m, k] (row stride ldx); y: f32 [m, n] (row stride ldy); ws: device
 * scratch of qmm_matmul_workspace_size(w, m) bytes (may be NULL for m <= 2,
 * where one kernel quantizes x in its prologue). m = 1..8 runs the decode
 * GEMV (replaces launch_mmvq_gguf_quantize_q8_1_f32 + launch_mmvq_gguf_*_f32_plain);
 * larger m runs the GEMM path (replaces launch_mmq_gguf_*). */
int qmm_matmul(const qmm_qtensor *w, const float *x, int64_t m, int64_t ldx, float *y, int64_t ldy,
               void *ws, size_t ws_bytes, void *stream);

/* qmm_matmul without a caller workspace, for callers that cannot allocate
 * (code under stream capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The workspace is a
 * library-held device array of QMM_NOALLOC_SCRATCH_BYTES per GPU, resolved at
 * set-up (qmm_init(device), else the first call on a device); the call itself
 * allocates nothing. Calls whose qmm_matmul_workspace_size(w, m) exceeds it
 * fail with QMM_ERR_INVALID. All calls on one GPU share the array: calls that
 * overlap on one GPU (other streams, other threads) race, so order them on
 * one stream. Results equal qmm_matmul's with a workspace of that size. */
#define QMM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int qmm_matmul_noalloc(const qmm_qtensor *w, const float *x, int64_t m, int64_t ldx, float *y, int64_t ldy,
                       void *stream);

/* `count` (1..8) QMatMul::forward calls on one input in a single launch:
 * y[j] = x . W[j]^T for weights of one dtype and k (e.g. a layer's q/k/v and
 * gate/up projections, which the reference engine runs as separate
 * QuantizedLinear::forward calls on the same activation, llama.rs:1066-1092,
 * 1386-1391). ldy[j] is the row stride of y[j]; ws: at least
 * qmm_matmul_workspace_size(w[0], m) bytes. For m > 8 the GEMMs of narrow
 * weights split K over more workgroups and need room for f32 partials: a
 * job whose split does not fit the workspace runs unsplit (same block dots,
 * another f32 summation order), so size ws as the largest over the weights
 * for the same results as separate qmm_matmul calls. */
int qmm_matmul_multi(const qmm_qtensor *const *w, int count, const float *x, int64_t m, int64_t ldx,
                     float *const *y, const int64_t *ldy, void *ws, size_t ws_bytes, void *stream);

/* Bytes of workspace the pre-quantized entry points below need for m
 * activation rows: 0 for m <= 8 (the GEMV reads the GGML blocks as they are);
 * for m > 8 the GEMM's activation planes plus, when the weight's output tiles
 * cover fewer than half the CUs, f32 split-K partials. The workspace is the
 * caller's: calls on different streams need different workspaces. */
size_t qmm_matmul_q_workspace_size(const qmm_qtensor *w, int64_t m);

/* The same with activations already quantized (xq: m rows of vec-dot blocks,
 * as produced by qmm_quantize_rows). For m > 8 the rows are rearranged for
 * the GEMM into `ws` (qmm_matmul_q_workspace_size(w, m) bytes; NULL allowed
 * for m <= 8). A workspace smaller than the planes is an error; one that holds
 * the planes but not the split-K partials runs the GEMM unsplit (same block
 * dots, another f32 summation order). */
int qmm_matmul_q(const qmm_qtensor *w, const void *xq, int64_t m, float *y, int64_t ldy, void *ws, size_t ws_bytes,
                 void *stream);

/* qmm_matmul_multi with activations already quantized (xq as for
 * qmm_matmul_q): `count` (1..8) weights of one k in one launch for m <= 8
 * (one GEMM per weight for larger m, all using `ws`, sized as the largest
 * qmm_matmul_q_workspace_size over the weights). The weights share one
 * dtype, or mix Q4_K and Q6_K (both multiply Q8_K activations): one launch at
 * m = 1, one per dtype otherwise. */
int qmm_matmul_multi_q(const qmm_qtensor *const *w, int count, const void *xq, int64_t m, float *const *y,
                       const int64_t *ldy, void *ws, size_t ws_bytes, void *stream);

/* qmm_matmul_q with an optional residual add (accumulate != 0: y += result;
 * then m <= 8). */
int qmm_matmul_q_ex(const qmm_qtensor *w, const void *xq, int64_t m, float *y, int64_t ldy, int accumulate,
                    void *ws, size_t ws_bytes, void *stream);

/* Debug entry: exact int32 block dots of every (activation row, weight row,
 * super-block), computed by the same kernel that qmm_matmul_q runs (the GEMV
 * for m <= 8, the MFMA GEMM for m > 8).
 * dots: device int32 [m, n, k/block_size, per] with per = 2 for Q4K
 * (isum_d = sum_j sc_j*sum q4*q8, isum_m = sum_j m_j*(bsum_2j + bsum_2j+1))
 * and per = 1 for Q6K (sum_j sc_j*sum (q6-32)*q8) and Q8_0 (sum qw*qx).
 * y receives the f32 outputs as qmm_matmul_q would. For m > 8, k must be a
 * multiple of 256 and ws holds qmm_matmul_q_workspace_size(w, m) bytes. */
int qmm_block_dots(const qmm_qtensor *w, const void *xq, int64_t m, float *y, int64_t ldy,
                   int32_t *dots, void *ws, size_t ws_bytes, void *stream);

/* Several QMatMul::forward calls at m = 1 on two independent input rows, in
 * one launch: weight w[i] (count 1..16, all Q4_K or all Q6_K, at most eight
 * per group, k <= 16384) multiplies the f32 row x[group[i]] (group 0 or 1;
 * the row's length is the k of that group's weights) into y[i] (w[i]->n
 * floats). Each group's row is quantized to Q8_K in the launch's prologue
 * as QMatMul::forward quantizes it, and every output equals qmm_matmul's on
 * that weight and row bit for bit. The launch's CUs are split between the
 * groups by their weight bytes, so independent GEMVs (e.g. one decoder
 * layer's projections of two different rows) stream with one ramp-up and one
 * drain instead of one per launch. No counterpart in the reference (its
 * launcher takes one weight). */
int qmm_matmul_grouped(const qmm_qtensor *const *w, const int *group, int count, const float *const *x,
                       float *const *y, void *stream);

/* QMatMul::forward for 1..8 weights (same k; one dtype, or Q4_K and Q6_K
 * together as for qmm_matmul_multi_q, e.g. a Q4_K_M layer's q, k and v) on
 * one input, with the decoder's neighbouring ops folded in: when norm_weight
 * is non-NULL the input rows are first RMS-normalised, x / sqrt(mean(x^2) + eps) * norm_weight
 * (rms_norm, crates/llm/candle-llm/src/primitives/nn.rs:22-31; fused into the
 * quantization prologue for m <= 2), and when `accumulate` is set the result
 * is added to y (the residual add of llama.rs:958-975). ws: device scratch of
 * qmm_matmul_ex_workspace_size(w[j], m, norm_weight != NULL) bytes, the
 * largest over the weights (m > 2 runs one pass per dtype). */
int qmm_matmul_ex(const qmm_qtensor *const *w, int count, const float *x, int64_t m, int64_t ldx,
                  const float *norm_weight, float eps, int accumulate, float *const *y, const int64_t *ldy,
                  void *ws, size_t ws_bytes, void *stream);
size_t qmm_matmul_ex_workspace_size(const qmm_qtensor *w, int64_t m, int normalize);

/* The gated feed-forward block of m rows (LlamaMlp::forward, SwiGLU,
 * llama.rs:1385-1392, after the block's RMSNorm, nn.rs:22-31): with n = x
 * RMS-normalised by norm_weight (or x itself when norm_weight is NULL),
 * y (+)= down(silu(gate(n)) * up(n)); y may be x (the residual add). gate and
 * up share shape and k; down's k is their n; every weight Q4_K or Q6_K. At
 * m > 8 the gate and up GEMMs leave their split-K partials unsummed and one
 * launch sums them (in split order), forms silu(g) * u and writes the down
 * GEMM's Q8_K planes: the same values as qmm_matmul_ex, qmm_silu_mul and
 * qmm_matmul_ex in sequence, in three launches fewer. m <= 8 runs those
 * GEMV calls. ws: qmm_ffn_workspace_size(gate, up, down, m, norm_weight !=
 * NULL) bytes. */
int qmm_ffn(const qmm_qtensor *gate, const qmm_qtensor *up, const qmm_qtensor *down, const float *x, int64_t m,
            int64_t ldx, const float *norm_weight, float eps, int accumulate, float *y, int64_t ldy, void *ws,
            size_t ws_bytes, void *stream);
size_t qmm_ffn_workspace_size(const qmm_qtensor *gate, const qmm_qtensor *up, const qmm_qtensor *down, int64_t m,
                              int normalize);

/* The attention projections of m prompt rows with RoPE and the KV append
 * (LlamaAttention::project and the cache update, llama.rs:1066-1114; apply_rope,
 * rope.rs:289-323; kv_cache.rs:107-111): q / k / v = wq / wk / wv applied to
 * x RMS-normalised by norm_weight (or x itself when NULL); the rows at
 * positions first .. first + m - 1 are rotated with the cos/sin tables
 * [max_seq][head_dim]; rotated q goes to q (row stride ldq), rotated k and v to
 * the caches [kv_heads][max_seq][head_dim]. Weights Q4_K or Q6_K of one k. At
 * m > 8 the three GEMMs leave their split-K partials unsummed and one launch
 * sums them (in split order), rotates and appends: the same values as
 * qmm_matmul_ex then qmm_rope_kv_append_n, in three launches fewer. m <= 8
 * runs those two calls. ws: qmm_qkv_rope_kv_append_n_workspace_size(wq, wk,
 * wv, m, norm_weight != NULL) bytes. */
int qmm_qkv_rope_kv_append_n(const qmm_qtensor *wq, const qmm_qtensor *wk, const qmm_qtensor *wv, const float *x,
                             int64_t m, int64_t ldx, const float *norm_weight, float eps, const float *cos_t,
                             const float *sin_t, int64_t first, float *q, int64_t ldq, float *kcache,
                             float *vcache, int heads, int kv_heads, int head_dim, int max_seq, void *ws,
                             size_t ws_bytes, void *stream);
size_t qmm_qkv_rope_kv_append_n_workspace_size(const qmm_qtensor *wq, const qmm_qtensor *wk, const qmm_qtensor *wv,
                                               int64_t m, int normalize);

/* ---- decode step of a Llama-style decoder (f32 ops around the matmuls) ---- */

/* RMSNorm of m rows: out = x / sqrt(mean(x^2) + eps) * w (nn.rs:22-31). */
int qmm_rms_norm(const float *x, int64_t m, int64_t k, int64_t ldx, const float *w, float eps, float *out,
                 int64_t ldo, void *stream);

/* x[0:hidden) = table[tokens[pos[0]]] (dense f32 embedding rows [vocab][ld]).
 * A token id outside [0, vocab) reads no table row and writes a NaN row. */
int qmm_embed_rows(const float *table, int64_t ld, int64_t vocab, const int32_t *tokens, const int32_t *pos,
                   float *x, int64_t hidden, void *stream);

/* In place NeoX RoPE of q [heads][head_dim] and k [kv_heads][head_dim] at
 * position pos[0] with cos/sin tables [max_seq][head_dim] (cat(freqs, freqs)),
 * then k and v are appended to the caches [kv_heads][max_seq][head_dim]
 * (apply_rope, rope.rs:289-323; KV concat, kv_cache.rs:107-111). */
int qmm_rope_kv_append(float *q, float *k, const float *v, const float *cos_t, const float *sin_t,
                       const int32_t *pos, float *kcache, float *vcache, int heads, int kv_heads, int head_dim,
                       int max_seq, void *stream);

/* Workspace bytes of the two attention calls below (0 for an unsupported
 * geometry): heads % kv_heads == 0, heads / kv_heads <= 8, head_dim in
 * {64, 128, 256}, 1 <= max_seq <= 1048576. The workspace starts with one
 * completion counter per kv head (a 256-byte-aligned region), then per-chunk
 * partial results; it must be zero before its first use, and every call
 * leaves the counters at zero. Calls that share a workspace must not run
 * concurrently; calls with workspaces of their own may run on concurrent
 * streams. */
size_t qmm_decode_attention_workspace_size(int heads, int kv_heads, int head_dim, int max_seq);

/* One query per head against cache positions 0..pos[0]: out[h] =
 * softmax(q[h] . K^T * scale) . V with kv head h / (heads / kv_heads)
 * (repeat_kv + sdpa_eager, attention.rs:59-68, 154-186). q is already
 * rotated and the cache already holds position pos[0]. */
int qmm_decode_attention(const float *q, const float *kcache, const float *vcache, const int32_t *pos,
                         float *out, int heads, int kv_heads, int head_dim, int max_seq, float scale, void *ws,
                         size_t ws_bytes, void *stream);

/* qmm_rope_kv_append followed by qmm_decode_attention in one launch: q, k
 * are the unrotated projections (left unchanged), the rotated k and v are
 * written to position pos[0] of the caches, out as qmm_decode_attention. */
int qmm_decode_rope_attention(const float *q, const float *k, const float *v, const float *cos_t,
                              const float *sin_t, const int32_t *pos, float *kcache, float *vcache, float *out,
                              int heads, int kv_heads, int head_dim, int max_seq, float scale, void *ws,
                              size_t ws_bytes, void *stream);

/* qmm_decode_rope_attention that also warms the caches for the one-row GEMV
 * launches that follow it in the decode step (the o projection, then
 * gate/up). The attention occupies half the CUs and almost none of the HBM
 * bandwidth; extra workgroups of the same launch load the first warm_rows[l]
 * rows per wave of launch l, each into the L2 of the XCD whose workgroup of
 * that launch will read them (a dispatch deals workgroups to the XCDs
 * round-robin, the same way for every launch). warm[i] (warm_count 0..3,
 * Q4_K / Q6_K) are the launches' weights in launch order, warm_launch[i] the
 * index of the launch weight i belongs to (non-decreasing); those launches
 * are fused one-row GEMVs (qmm_matmul_ex at m = 1). The loads write nothing,
 * so the results equal qmm_decode_rope_attention's. No counterpart in the
 * reference (a scheduling aid of this backend's decode step). */
int qmm_decode_rope_attention_warm(const float *q, const float *k, const float *v, const float *cos_t,
                                   const float *sin_t, const int32_t *pos, float *kcache, float *vcache,
                                   float *out, int heads, int kv_heads, int head_dim, int max_seq, float scale,
                                   void *ws, size_t ws_bytes, const qmm_qtensor *const *warm,
                                   const int *warm_launch, int warm_count, const int *warm_rows, void *stream);

/* Batched prefill: the same per-layer operations over `count` prompt rows at
 * positions first .. first + count - 1 (CausalLm::forward over a prompt with
 * seq_len > 1 and the causal mask, llama.rs:410-433, 654-725; causal sdpa,
 * attention.rs:154-186). Rows are row-major with the given strides. */

/* x[i] = table[tokens[first + i]] for i < count (CausalLm embed, llama.rs:397-408);
 * token ids outside [0, vocab) give NaN rows as in qmm_embed_rows. */
int qmm_embed_rows_n(const float *table, int64_t ld, int64_t vocab, const int32_t *tokens, int64_t first,
                     int64_t count, float *x, int64_t hidden, void *stream);

/* qmm_rope_kv_append for rows i < count at positions first + i: q and k
 * rows rotated in place, k and v written to the caches at those positions. */
int qmm_rope_kv_append_n(float *q, float *k, const float *v, int64_t ldq, int64_t ldk, int64_t ldv,
                         const float *cos_t, const float *sin_t, int64_t first, int64_t count, float *kcache,
                         float *vcache, int heads, int kv_heads, int head_dim, int max_seq, void *stream);

/* Causal GQA attention of rows i < count: query row i (already rotated, at
 * position first + i) against cache positions 0 ..= first + i, out row i =
 * softmax(q . K^T * scale) . V per head (geometry as qmm_decode_attention). */
int qmm_prefill_attention(const float *q, int64_t ldq, const float *kcache, const float *vcache, int64_t first,
                          int64_t count, float *out, int64_t ldo, int heads, int kv_heads, int head_dim, int max_seq,
                          float scale, void *stream);

/* qmm_prefill_attention followed by qmm_matmul_ex(&wo, 1, ...) with accumulate:
 * x[i] += att[i] . wo^T for the count prompt rows (LlamaAttention::forward's
 * o_proj and the decoder layer's residual add, llama.rs:1115-1120, 654-725),
 * bit for bit. Where the o GEMM takes Q8_K planes (count > 8, a Q4_K / Q6_K
 * weight) and heads / kv_heads * head_dim is a multiple of 256, the attention
 * launch writes those planes itself. ws: device scratch of
 * qmm_prefill_attention_o_workspace_size(wo, count) bytes. */
int qmm_prefill_attention_o(const float *q, int64_t ldq, const float *kcache, const float *vcache, int64_t first,
                            int64_t count, int heads, int kv_heads, int head_dim, int max_seq, float scale,
                            const qmm_qtensor *wo, float *x, int64_t ldx, void *ws, size_t ws_bytes, void *stream);
size_t qmm_prefill_attention_o_workspace_size(const qmm_qtensor *wo, int64_t count);

/* h = silu(g) * u over n elements, f32 (LlamaMlp::forward, llama.rs:1386-1391). */
int qmm_silu_mul(const float *g, const float *u, float *h, int64_t n, void *stream);

/* hq = Q8_K(silu(g) * u) for rows x k (k a multiple of 256), the down
 * projection's activation (LlamaMlp::forward, llama.rs:1386-1391). */
int qmm_silu_mul_quantize(const float *g, const float *u, int64_t rows, int64_t k, int64_t ld, void *hq,
                          void *stream);

/* The down projection of one token with its activation formed in the same
 * launch: y (+)= QMatMul::forward(silu(g) * u), i.e. qmm_silu_mul_quantize
 * followed by qmm_matmul_q_ex, with the Q8_K quantization done in the GEMV
 * prologue (LlamaMlp::forward, llama.rs:1386-1391: down(silu(gate) * up)).
 * g, u: f32 [w->k] (k-quant weights, k a multiple of 256); y: f32 [w->n];
 * accumulate != 0 adds to y. Results are identical to the two-call form. */
int qmm_silu_mul_matmul(const qmm_qtensor *w, const float *g, const float *u, float *y, int accumulate,
                        void *stream);

/* Workspace bytes of qmm_greedy_advance; the first 256 bytes are a counter
 * with the same zero-before-first-use contract as the attention workspace. */
size_t qmm_greedy_workspace_size(int64_t n);

/* Greedy step end on the device: tokens[pos+1] = argmax(logits) (lowest index
 * on ties, argmax_device, sampler.rs:216-219; a NaN counts as the largest
 * value, the first NaN wins, as torch.argmax) unless pos+1 < prompt_len (the
 * slot still holds a prompt token); then pos[0] += 1. `capacity` is the
 * length of tokens (and of the KV cache): once pos+1 reaches it the call
 * writes nothing and pos stays, so a step replayed too often never writes
 * out of bounds. */
int qmm_greedy_advance(const float *logits, int64_t n, int32_t *tokens, int64_t capacity, int32_t *pos,
                       int prompt_len, void *ws, size_t ws_bytes, void *stream);

/* ---- mixture of experts (MoeMlp::forward, crates/llm/candle-llm/src/models/llama.rs:1416-1487) ---- */

/* Routing on the device: logits f32 [tokens, experts] -> softmax -> top-k
 * (renormalised over the selected experts when `renormalize`). Outputs are
 * device int32/f32 arrays: counts[experts], offsets[experts + 1] (exclusive
 * prefix), and tokens*topk (token, weight) pairs grouped by expert in
 * increasing expert order (pair_token, pair_weight); token_pairs[t*topk + s]
 * lists token t's pairs in increasing expert order. Replaces the host-side
 * top-k of llama.rs:1426-1451. Limits: tokens <= 4096, tokens*topk <= 8192. */
int qmm_moe_route(const float *logits, int64_t tokens, int experts, int topk, int renormalize,
                  int32_t *counts, int32_t *offsets, int32_t *pair_token, float *pair_weight,
                  int32_t *token_pairs, void *stream);
/* qmm_moe_route with MoeMlp::forward's other weight branch (llama.rs:1436-1447):
 * renormalize (norm_topk_prob) gives p / sum over the selection; otherwise each
 * weight is p * routed_scaling_factor (DeepSeek's routed_scaling_factor; 1.0
 * for Qwen2-MoE). qmm_moe_route is this with routed_scaling_factor = 1. */
int qmm_moe_route_ex(const float *logits, int64_t tokens, int experts, int topk, int renormalize,
                     float routed_scaling_factor, int32_t *counts, int32_t *offsets, int32_t *pair_token,
                     float *pair_weight, int32_t *token_pairs, void *stream);

/* Expert-grouped GEMV (replaces moe_gemm_gguf, ffi.rs:25-39): w[j] (count 1..2)
 * are stacked expert weights [experts*N, K] of one dtype; xq holds `pairs`
 * rows of vec-dot blocks grouped by expert (counts/offsets as produced by
 * qmm_moe_route); y[j] receives [pairs, N] f32. An active expert's weights
 * are streamed once per 8 of its tokens; experts without tokens read nothing.
 * Every counts[e] must be <= pairs (the launch is sized for that bound). */
int qmm_moe_gemv(const qmm_qtensor *const *w, int count, int experts, const void *xq, int64_t pairs,
                 const int32_t *counts, const int32_t *offsets, float *const *y, void *stream);

/* Expert-grouped prefill GEMM (replaces the grouped prefill launcher
 * moe/moe_wmma_gguf.cu:124-354 and the per-expert QMatMul::forward over
 * gathered rows of MoeMlp::forward, llama.rs:1455-1474): x holds `pairs` f32
 * rows (stride ldx) grouped by expert (counts/offsets as from
 * qmm_moe_route); y[j] receives [pairs, N] f32 with N = rows / experts. The
 * rows are quantized once (Q8_K / Q8_0, as QMatMul::forward does), then each
 * expert's rows go through the int8 MFMA GEMM against its weight slice.
 * max_rows bounds every count (e.g. the token count for top-k routing).
 * Outputs equal qmm_matmul's GEMM path on each expert's rows bit for bit.
 * ws: qmm_moe_gemm_workspace_size(w[0], pairs) bytes; k % 256 == 0. */
size_t qmm_moe_gemm_workspace_size(const qmm_qtensor *w, int64_t pairs);
int qmm_moe_gemm(const qmm_qtensor *const *w, int count, int experts, const float *x, int64_t pairs, int64_t ldx,
                 int64_t max_rows, const int32_t *counts, const int32_t *offsets, float *const *y, void *ws,
                 size_t ws_bytes, void *stream);

/* The whole expert FFN at decode batch sizes: x f32 [tokens, hidden] (row
 * stride ldx), router logits f32 [tokens, experts], stacked gate/up
 * [experts*ffn, hidden] and down [experts*hidden, ffn] weights; out f32
 * [tokens, hidden] (row stride ldo) = sum over each token's top-k experts, in
 * increasing expert order, of weight * down(silu(gate(x)) * up(x)).
 * Any token count: a list longer than the routing limit (min(4096, 8192 /
 * topk) tokens) runs as consecutive chunks of that many tokens, in stream
 * order through the same workspace; tokens are routed and combined
 * independently, so the result is the whole list's.
 * ws: device scratch of qmm_moe_ffn_workspace_size() bytes (one chunk's). */
size_t qmm_moe_ffn_workspace_size(const qmm_qtensor *gate, const qmm_qtensor *down, int64_t tokens,
                                  int experts, int topk);
int qmm_moe_ffn(const float *x, int64_t tokens, int64_t ldx, const float *logits, int experts, int topk,
                const qmm_qtensor *gate, const qmm_qtensor *up, const qmm_qtensor *down, float *out,
                int64_t ldo, void *ws, size_t ws_bytes, void *stream);

/* The whole of MoeMlp::forward (models/llama.rs:1416-1487), of which
 * qmm_moe_ffn is the Mixtral case (norm_topk_prob, no shared expert):
 *   * routed weights as qmm_moe_route_ex (norm_topk_prob != 0: renormalised;
 *     else times routed_scaling_factor);
 *   * an optional always-on shared expert (shared_gate / shared_up /
 *     shared_down: a dense-row gated MLP, [Fs, hidden] / [Fs, hidden] /
 *     [hidden, Fs], as qmm_ffn runs it over every token), added after the
 *     routed sum; with shared_gate_weight (f32 [hidden] on the device) it is
 *     first scaled per token by sigmoid(x . shared_gate_weight) (Qwen2-MoE),
 *     without it added ungated (DeepSeek-V2). All three shared weights NULL: no
 *     shared expert.
 * ws: qmm_moe_ffn_ex_workspace_size(...) bytes with the same shared weights. */
size_t qmm_moe_ffn_ex_workspace_size(const qmm_qtensor *gate, const qmm_qtensor *down, int64_t tokens,
                                     int experts, int topk, const qmm_qtensor *shared_gate,
                                     const qmm_qtensor *shared_up, const qmm_qtensor *shared_down);
int qmm_moe_ffn_ex(const float *x, int64_t tokens, int64_t ldx, const float *logits, int experts, int topk,
                   int norm_topk_prob, float routed_scaling_factor, const qmm_qtensor *gate,
                   const qmm_qtensor *up, const qmm_qtensor *down, const qmm_qtensor *shared_gate,
                   const qmm_qtensor *shared_up, const qmm_qtensor *shared_down,
                   const float *shared_gate_weight, float *out, int64_t ldo, void *ws, size_t ws_bytes,
                   void *stream);

/* ---------------------------------------------------------------------------
 * GGUF files (llama.cpp's single-file model container, spec v2/v3).
 * Replaces the reference's GgufFile (crates/llm/mlx-llm/src/gguf/reader.rs:
 * GgufFile::open/parse :188-278, meta/meta_str/meta_u64/meta_f64 :281-303,
 * tensor_data :307-328; MetaValue::as_u64/as_i64/as_f64/as_str :73-131) and
 * candle's gguf_file::Content::{read, tensor} at the engine's call sites
 * (crates/llm/candle-llm/src/gguf.rs:68, 101-103). Unlike the engine, which
 * dequantizes every tensor and re-quantizes it, qmm_gguf_load_qtensor puts
 * a quantized tensor's blocks straight into a device QTensor.
 * ------------------------------------------------------------------------- */
typedef struct qmm_gguf qmm_gguf;

/* Open a file (memory-mapped, read only) or an in-memory image (copied).
 * Errors: bad magic, version other than 2 or 3 (QMM_ERR_UNSUPPORTED), counts
 * above 2^20, truncated tables, tensors of 0 or more than 4 dims, nested
 * arrays, unknown value types, a data section past the end of the file. */
int qmm_gguf_open(const char *path, qmm_gguf **out);
int qmm_gguf_open_memory(const void *bytes, size_t len, qmm_gguf **out);
void qmm_gguf_close(qmm_gguf *g);

int qmm_gguf_version(const qmm_gguf *g);
/* general.alignment when it is an integer (>= 1), else 32. */
uint64_t qmm_gguf_alignment(const qmm_gguf *g);
int64_t qmm_gguf_tensor_count(const qmm_gguf *g);
int64_t qmm_gguf_metadata_count(const qmm_gguf *g);

/* Index of a tensor / metadata key (-1 if absent; a repeated key keeps its last value). */
int64_t qmm_gguf_find_tensor(const qmm_gguf *g, const char *name);
int64_t qmm_gguf_meta_find(const qmm_gguf *g, const char *key);

/* Tensor i: name (owned by g), dims, shape in torch order (the GGML ne order
 * reversed: [out, in] for a linear weight; unused entries 0), GGML type tag
 * and byte offset within the data section. */
int qmm_gguf_tensor_info(const qmm_gguf *g, int64_t i, const char **name, int *ndims, int64_t *shape,
                         int *ggml_type, uint64_t *offset);
/* (elements, bytes) per block of a GGML type tag (dequant.rs:86-140). */
int qmm_gguf_type_size(int ggml_type, uint64_t *block_elems, uint64_t *block_bytes);
/* Host pointer to tensor i's bytes inside the file and their length
 * (elements / block_elems * block_bytes); out-of-range data is an error. */
int qmm_gguf_tensor_data(const qmm_gguf *g, int64_t i, const void **data, size_t *bytes);

/* Metadata entry i: key, value type (GGUF tags 0..12; 9 = array), element
 * type (arrays) and count (1 for scalars). Values: elem = -1 for a scalar,
 * else the array element. u64 takes unsigned integers, non-negative signed
 * ones and bools; i64 any integer; f64 f32/f64; string a pointer into the
 * file (not NUL-terminated) and its length. A type mismatch is an error. */
int qmm_gguf_meta_info(const qmm_gguf *g, int64_t i, const char **key, int *type, int *elem_type,
                       uint64_t *count);
int qmm_gguf_meta_u64(const qmm_gguf *g, int64_t i, int64_t elem, uint64_t *v);
int qmm_gguf_meta_i64(const qmm_gguf *g, int64_t i, int64_t elem, int64_t *v);
int qmm_gguf_meta_f64(const qmm_gguf *g, int64_t i, int64_t elem, double *v);
int qmm_gguf_meta_string(const qmm_gguf *g, int64_t i, int64_t elem, const char **s, uint64_t *len);

/* Resident load of a 2-D Q8_0 / Q4_K / Q6_K tensor into a device QTensor
 * (QStorage::from_data + QTensor::new, candle-gen/src/quant/repack.rs:202-203),
 * on the current device, synchronous. unpermute_heads > 0 undoes llama.cpp's
 * q/k row order per head on the quantized rows (unpermute_qk, candle-llm
 * gguf.rs:333-356: torch row k * hd/2 + j of a head is GGUF row 2j + k). */
int qmm_gguf_load_qtensor(const qmm_gguf *g, int64_t i, int unpermute_heads, void *stream, qmm_qtensor **out);

/* Measurement aid, no counterpart in the reference: a plain streaming read
 * of `bytes` (a multiple of 16) at `data` on the device, the ceiling a
 * weight-streaming launch of the same size is measured against. variant:
 * 0 grid-stride with 4 loads in flight per thread, 1 grid-stride with 8,
 * 2 one contiguous chunk per workgroup with 8 nontemporal loads in flight
 * (no variant is fastest at every size). wgs_per_cu workgroups of 256
 * threads per CU (0: 8; at most 64); `sink` (one word) is written only if
 * the folded data equals a fixed constant. */
int qmm_stream_read(const void *data, size_t bytes, uint32_t *sink, int variant, int wgs_per_cu, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* QMM_H */

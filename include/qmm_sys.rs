//! Raw bindings of `libqmm.so` (include/qmm.h): the `-sys` layer a Rust engine adds next to
//! its CUDA launchers (the reference's pattern: vendor/candle-kernels/src/ffi.rs:4-631, one
//! `extern "C"` block of the launcher signatures), followed by a thin safe layer over the entry
//! points the quantized-matmul path calls (QTensor / QMatMul in
//! crates/llm/candle-llm/src/primitives/quant.rs:17-43).
//!
//! Every function mirrors its C declaration one to one (same name, order and meaning of the
//! arguments); pointers are device pointers unless the C comment says host, and `stream` is a
//! `hipStream_t` (null = the default stream). Each call returns a status (`QMM_OK` = 0) and
//! `qmm_last_error()` holds the calling thread's message. Link with `-lqmm` (the library embeds
//! its gfx950 code object and needs only libamdhip64 beside it).
#![allow(non_camel_case_types, clippy::missing_safety_doc)]

use std::ffi::{CStr, CString};
use std::os::raw::{c_char, c_int, c_void};

pub const QMM_OK: c_int = 0;
pub const QMM_ERR_INVALID: c_int = 1;
pub const QMM_ERR_HIP: c_int = 2;
pub const QMM_ERR_NO_KERNEL: c_int = 3;
pub const QMM_ERR_UNSUPPORTED: c_int = 4;
pub const QMM_ERR_OOM: c_int = 5;

/// GGML dtype tags (GGUF numbering).
pub const QMM_F32: c_int = 0;
pub const QMM_F16: c_int = 1;
pub const QMM_BF16: c_int = 30;
pub const QMM_Q8_0: c_int = 8;
pub const QMM_Q4K: c_int = 12;
pub const QMM_Q6K: c_int = 14;
pub const QMM_Q8K: c_int = 15;

/// Workspace bytes held per GPU by `qmm_matmul_noalloc`.
pub const QMM_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

/// Opaque device QTensor handle.
#[repr(C)]
pub struct QmmQTensor {
    _private: [u8; 0],
}

/// Opaque parsed GGUF file.
#[repr(C)]
pub struct QmmGguf {
    _private: [u8; 0],
}

#[link(name = "qmm")]
extern "C" {
    /// Last error message of the calling thread ("" if none).
    pub fn qmm_last_error() -> *const c_char;

    /// Load the kernel code object on `device` (optional: every entry point loads it
    /// lazily for the current device).
    pub fn qmm_init(device: c_int) -> c_int;

    /// Re-read the QMM_* tuning overrides from the environment (read once, at the first call,
    /// and then only here).
    pub fn qmm_reload_tuning();

    /// GGML geometry: elements per block, bytes per block, and the activation type a
    /// weight type multiplies against (Q8_0 -> Q8_0, Q4K/Q6K -> Q8K). -1 if unknown.
    /// (GgmlDType::block_size / type_size / vec_dot_type.)
    pub fn qmm_block_size(dtype: c_int) -> c_int;

    pub fn qmm_type_size(dtype: c_int) -> c_int;

    pub fn qmm_vec_dot_type(dtype: c_int) -> c_int;

    /// QTensor::new(QStorage::from_data(bytes, device, dtype), (n, k)).
    /// `bytes` holds n*k/block_size GGML blocks, row-major over n then k, on the
    /// host (bytes_on_device = 0) or on the current device (= 1). The bytes are
    /// copied into the handle's own device layout; the caller keeps `bytes`.
    pub fn qmm_qtensor_from_ggml(
        dtype: c_int, n: i64, k: i64, bytes: *const c_void, bytes_on_device: c_int, stream: *mut c_void,
        out: *mut *mut QmmQTensor
    ) -> c_int;

    /// QTensor::quantize(&Tensor f32 [n, k], dtype) computed on the device:
    /// `w` is a device pointer to n*k f32 (row-major). The result's GGML bytes
    /// equal those of candle's CPU from_float for the same input.
    pub fn qmm_qtensor_quantize(
        dtype: c_int, n: i64, k: i64, w: *const f32, stream: *mut c_void, out: *mut *mut QmmQTensor
    ) -> c_int;

    /// QTensor::dequantize: n*k f32 into the device buffer `dst`.
    pub fn qmm_qtensor_dequantize(t: *const QmmQTensor, dst: *mut f32, stream: *mut c_void) -> c_int;

    /// qmm_qtensor_dequantize to a dense [n, k] of out_dtype QMM_F32, QMM_F16 or
    /// QMM_BF16 (each value rounded to nearest even from its f32 dequantization):
    /// candle's QTensor::dequantize_f16 and the dequant-dense matmul strategy's
    /// weight.dequantize(device).to_dtype(x.dtype) (candle-gen/src/quant/mod.rs:
    /// 515-533; QMatMul::forward_via_f16 at candle-gen-lens/src/text_encoder.rs:
    /// 518-529).
    pub fn qmm_qtensor_dequantize_to(
        t: *const QmmQTensor, dst: *mut c_void, out_dtype: c_int, stream: *mut c_void
    ) -> c_int;

    /// Export the tensor as GGML block bytes (qmm_qtensor_ggml_bytes() of them) into
    /// `dst` on the host (dst_on_device = 0, synchronous) or the device (= 1).
    pub fn qmm_qtensor_to_ggml(
        t: *const QmmQTensor, dst: *mut c_void, dst_on_device: c_int, stream: *mut c_void
    ) -> c_int;

    /// Shape and dtype; size of the GGML byte image.
    pub fn qmm_qtensor_info(t: *const QmmQTensor, dtype: *mut c_int, n: *mut i64, k: *mut i64) -> c_int;

    pub fn qmm_qtensor_ggml_bytes(t: *const QmmQTensor) -> usize;

    /// Free a handle and its device memory (NULL is ignored).
    pub fn qmm_qtensor_free(t: *mut QmmQTensor);

    /// VecDotType::from_float on the device (replaces launch_mmvq_gguf_quantize_q8_1_f32,
    /// ffi.rs:412-419): x is f32 [m, k] with row stride ldx (elements); xq receives
    /// m rows of k/block_size blocks of `vdtype` (QMM_Q8_0 or QMM_Q8K), GGML bytes,
    /// contiguous. Bytes equal the CPU quantizer's for the same input.
    pub fn qmm_quantize_rows(
        vdtype: c_int, x: *const f32, m: i64, k: i64, ldx: i64, xq: *mut c_void, stream: *mut c_void
    ) -> c_int;

    /// Bytes of workspace qmm_matmul needs for m activation rows (for m > 8: the
    /// GEMM's quantized activation planes plus, when the weight's output tiles
    /// cover fewer than half the CUs, f32 split-K partials).
    pub fn qmm_matmul_workspace_size(w: *const QmmQTensor, m: i64) -> usize;

    /// QMatMul::forward: y[i, j] = sum_k x[i, k] * W[j, k] for i < m, j < n, with x
    /// quantized to W's vec-dot type first (as Candle's CPU path does).
    /// x: f32 [m, k] (row stride ldx); y: f32 [m, n] (row stride ldy); ws: device
    /// scratch of qmm_matmul_workspace_size(w, m) bytes (may be NULL for m <= 2,
    /// where one kernel quantizes x in its prologue). m = 1..8 runs the decode
    /// GEMV (replaces launch_mmvq_gguf_quantize_q8_1_f32 + launch_mmvq_gguf_*_f32_plain);
    /// larger m runs the GEMM path (replaces launch_mmq_gguf_*).
    pub fn qmm_matmul(
        w: *const QmmQTensor, x: *const f32, m: i64, ldx: i64, y: *mut f32, ldy: i64, ws: *mut c_void,
        ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    pub fn qmm_matmul_noalloc(
        w: *const QmmQTensor, x: *const f32, m: i64, ldx: i64, y: *mut f32, ldy: i64, stream: *mut c_void
    ) -> c_int;

    /// `count` (1..8) QMatMul::forward calls on one input in a single launch:
    /// y[j] = x . W[j]^T for weights of one dtype and k (e.g. a layer's q/k/v and
    /// gate/up projections, which the reference engine runs as separate
    /// QuantizedLinear::forward calls on the same activation, llama.rs:1066-1092,
    /// 1386-1391). ldy[j] is the row stride of y[j]; ws: at least
    /// qmm_matmul_workspace_size(w[0], m) bytes. For m > 8 the GEMMs of narrow
    /// weights split K over more workgroups and need room for f32 partials: a
    /// job whose split does not fit the workspace runs unsplit (same block dots,
    /// another f32 summation order), so size ws as the largest over the weights
    /// for the same results as separate qmm_matmul calls.
    pub fn qmm_matmul_multi(
        w: *const *const QmmQTensor, count: c_int, x: *const f32, m: i64, ldx: i64, y: *const *mut f32,
        ldy: *const i64, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// Bytes of workspace the pre-quantized entry points below need for m
    /// activation rows: 0 for m <= 8 (the GEMV reads the GGML blocks as they are);
    /// for m > 8 the GEMM's activation planes plus, when the weight's output tiles
    /// cover fewer than half the CUs, f32 split-K partials. The workspace is the
    /// caller's: calls on different streams need different workspaces.
    pub fn qmm_matmul_q_workspace_size(w: *const QmmQTensor, m: i64) -> usize;

    /// The same with activations already quantized (xq: m rows of vec-dot blocks,
    /// as produced by qmm_quantize_rows). For m > 8 the rows are rearranged for
    /// the GEMM into `ws` (qmm_matmul_q_workspace_size(w, m) bytes; NULL allowed
    /// for m <= 8). A workspace smaller than the planes is an error; one that holds
    /// the planes but not the split-K partials runs the GEMM unsplit (same block
    /// dots, another f32 summation order).
    pub fn qmm_matmul_q(
        w: *const QmmQTensor, xq: *const c_void, m: i64, y: *mut f32, ldy: i64, ws: *mut c_void,
        ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// qmm_matmul_multi with activations already quantized (xq as for
    /// qmm_matmul_q): `count` (1..8) weights of one k in one launch for m <= 8
    /// (one GEMM per weight for larger m, all using `ws`, sized as the largest
    /// qmm_matmul_q_workspace_size over the weights). The weights share one
    /// dtype, or mix Q4_K and Q6_K (both multiply Q8_K activations): one launch at
    /// m = 1, one per dtype otherwise.
    pub fn qmm_matmul_multi_q(
        w: *const *const QmmQTensor, count: c_int, xq: *const c_void, m: i64, y: *const *mut f32,
        ldy: *const i64, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// qmm_matmul_q with an optional residual add (accumulate != 0: y += result;
    /// then m <= 8).
    pub fn qmm_matmul_q_ex(
        w: *const QmmQTensor, xq: *const c_void, m: i64, y: *mut f32, ldy: i64, accumulate: c_int,
        ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// Debug entry: exact int32 block dots of every (activation row, weight row,
    /// super-block), computed by the same kernel that qmm_matmul_q runs (the GEMV
    /// for m <= 8, the MFMA GEMM for m > 8).
    /// dots: device int32 [m, n, k/block_size, per] with per = 2 for Q4K
    /// (isum_d = sum_j sc_j*sum q4*q8, isum_m = sum_j m_j*(bsum_2j + bsum_2j+1))
    /// and per = 1 for Q6K (sum_j sc_j*sum (q6-32)*q8) and Q8_0 (sum qw*qx).
    /// y receives the f32 outputs as qmm_matmul_q would. For m > 8, k must be a
    /// multiple of 256 and ws holds qmm_matmul_q_workspace_size(w, m) bytes.
    pub fn qmm_block_dots(
        w: *const QmmQTensor, xq: *const c_void, m: i64, y: *mut f32, ldy: i64, dots: *mut i32,
        ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// QMatMul::forward for 1..8 weights (same k; one dtype, or Q4_K and Q6_K
    /// together as for qmm_matmul_multi_q, e.g. a Q4_K_M layer's q, k and v) on
    /// one input, with the decoder's neighbouring ops folded in: when norm_weight
    /// is non-NULL the input rows are first RMS-normalised, x / sqrt(mean(x^2) + eps) * norm_weight
    /// (rms_norm, crates/llm/candle-llm/src/primitives/nn.rs:22-31; fused into the
    /// quantization prologue for m <= 2), and when `accumulate` is set the result
    /// is added to y (the residual add of llama.rs:958-975). ws: device scratch of
    /// qmm_matmul_ex_workspace_size(w[j], m, norm_weight != NULL) bytes, the
    /// largest over the weights (m > 2 runs one pass per dtype).
    /// Several `QMatMul::forward` calls at m = 1 on two independent rows in one launch (results equal
    /// `qmm_matmul` on each weight bit for bit).
    pub fn qmm_matmul_grouped(
        w: *const *const QmmQTensor, group: *const c_int, count: c_int, x: *const *const f32,
        y: *const *mut f32, stream: *mut c_void
    ) -> c_int;

    pub fn qmm_matmul_ex(
        w: *const *const QmmQTensor, count: c_int, x: *const f32, m: i64, ldx: i64, norm_weight: *const f32,
        eps: f32, accumulate: c_int, y: *const *mut f32, ldy: *const i64, ws: *mut c_void, ws_bytes: usize,
        stream: *mut c_void
    ) -> c_int;

    pub fn qmm_matmul_ex_workspace_size(w: *const QmmQTensor, m: i64, normalize: c_int) -> usize;

    /// The gated feed-forward block of m rows (LlamaMlp::forward, SwiGLU,
    /// llama.rs:1385-1392, after the block's RMSNorm, nn.rs:22-31): with n = x
    /// RMS-normalised by norm_weight (or x itself when norm_weight is NULL),
    /// y (+)= down(silu(gate(n)) * up(n)); y may be x (the residual add). gate and
    /// up share shape and k; down's k is their n; every weight Q4_K or Q6_K. At
    /// m > 8 the gate and up GEMMs leave their split-K partials unsummed and one
    /// launch sums them (in split order), forms silu(g) * u and writes the down
    /// GEMM's Q8_K planes: the same values as qmm_matmul_ex, qmm_silu_mul and
    /// qmm_matmul_ex in sequence, in three launches fewer. m <= 8 runs those
    /// GEMV calls. ws: qmm_ffn_workspace_size(gate, up, down, m, norm_weight !=
    /// NULL) bytes.
    pub fn qmm_ffn(
        gate: *const QmmQTensor, up: *const QmmQTensor, down: *const QmmQTensor, x: *const f32, m: i64, ldx: i64,
        norm_weight: *const f32, eps: f32, accumulate: c_int, y: *mut f32, ldy: i64, ws: *mut c_void,
        ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    pub fn qmm_ffn_workspace_size(
        gate: *const QmmQTensor, up: *const QmmQTensor, down: *const QmmQTensor, m: i64, normalize: c_int
    ) -> usize;

    /// The attention projections of m prompt rows with RoPE and the KV append
    /// (LlamaAttention::project and the cache update, llama.rs:1066-1114; apply_rope,
    /// rope.rs:289-323; kv_cache.rs:107-111): q / k / v = wq / wk / wv applied to
    /// x RMS-normalised by norm_weight (or x itself when NULL); the rows at
    /// positions first .. first + m - 1 are rotated with the cos/sin tables
    /// [max_seq][head_dim]; rotated q goes to q (row stride ldq), rotated k and v to
    /// the caches [kv_heads][max_seq][head_dim]. Weights Q4_K or Q6_K of one k. At
    /// m > 8 the three GEMMs leave their split-K partials unsummed and one launch
    /// sums them (in split order), rotates and appends: the same values as
    /// qmm_matmul_ex then qmm_rope_kv_append_n, in three launches fewer. m <= 8
    /// runs those two calls. ws: qmm_qkv_rope_kv_append_n_workspace_size(wq, wk,
    /// wv, m, norm_weight != NULL) bytes.
    pub fn qmm_qkv_rope_kv_append_n(
        wq: *const QmmQTensor, wk: *const QmmQTensor, wv: *const QmmQTensor, x: *const f32, m: i64, ldx: i64,
        norm_weight: *const f32, eps: f32, cos_t: *const f32, sin_t: *const f32, first: i64, q: *mut f32, ldq: i64,
        kcache: *mut f32, vcache: *mut f32, heads: c_int, kv_heads: c_int, head_dim: c_int, max_seq: c_int,
        ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    pub fn qmm_qkv_rope_kv_append_n_workspace_size(
        wq: *const QmmQTensor, wk: *const QmmQTensor, wv: *const QmmQTensor, m: i64, normalize: c_int
    ) -> usize;

    /// RMSNorm of m rows: out = x / sqrt(mean(x^2) + eps) * w (nn.rs:22-31).
    pub fn qmm_rms_norm(
        x: *const f32, m: i64, k: i64, ldx: i64, w: *const f32, eps: f32, out: *mut f32, ldo: i64,
        stream: *mut c_void
    ) -> c_int;

    /// x[0:hidden) = table[tokens[pos[0]]] (dense f32 embedding rows [vocab][ld]).
    /// A token id outside [0, vocab) reads no table row and writes a NaN row.
    pub fn qmm_embed_rows(
        table: *const f32, ld: i64, vocab: i64, tokens: *const i32, pos: *const i32, x: *mut f32,
        hidden: i64, stream: *mut c_void
    ) -> c_int;

    /// In place NeoX RoPE of q [heads][head_dim] and k [kv_heads][head_dim] at
    /// position pos[0] with cos/sin tables [max_seq][head_dim] (cat(freqs, freqs)),
    /// then k and v are appended to the caches [kv_heads][max_seq][head_dim]
    /// (apply_rope, rope.rs:289-323; KV concat, kv_cache.rs:107-111).
    pub fn qmm_rope_kv_append(
        q: *mut f32, k: *mut f32, v: *const f32, cos_t: *const f32, sin_t: *const f32, pos: *const i32,
        kcache: *mut f32, vcache: *mut f32, heads: c_int, kv_heads: c_int, head_dim: c_int, max_seq: c_int,
        stream: *mut c_void
    ) -> c_int;

    /// Workspace bytes of the two attention calls below (0 for an unsupported
    /// geometry): heads % kv_heads == 0, heads / kv_heads <= 8, head_dim in
    /// {64, 128, 256}, 1 <= max_seq <= 1048576. The workspace starts with one
    /// completion counter per kv head (a 256-byte-aligned region), then per-chunk
    /// partial results; it must be zero before its first use, and every call
    /// leaves the counters at zero. Calls that share a workspace must not run
    /// concurrently; calls with workspaces of their own may run on concurrent
    /// streams.
    pub fn qmm_decode_attention_workspace_size(
        heads: c_int, kv_heads: c_int, head_dim: c_int, max_seq: c_int
    ) -> usize;

    /// One query per head against cache positions 0..pos[0]: out[h] =
    /// softmax(q[h] . K^T * scale) . V with kv head h / (heads / kv_heads)
    /// (repeat_kv + sdpa_eager, attention.rs:59-68, 154-186). q is already
    /// rotated and the cache already holds position pos[0].
    pub fn qmm_decode_attention(
        q: *const f32, kcache: *const f32, vcache: *const f32, pos: *const i32, out: *mut f32, heads: c_int,
        kv_heads: c_int, head_dim: c_int, max_seq: c_int, scale: f32, ws: *mut c_void, ws_bytes: usize,
        stream: *mut c_void
    ) -> c_int;

    /// qmm_rope_kv_append followed by qmm_decode_attention in one launch: q, k
    /// are the unrotated projections (left unchanged), the rotated k and v are
    /// written to position pos[0] of the caches, out as qmm_decode_attention.
    pub fn qmm_decode_rope_attention(
        q: *const f32, k: *const f32, v: *const f32, cos_t: *const f32, sin_t: *const f32, pos: *const i32,
        kcache: *mut f32, vcache: *mut f32, out: *mut f32, heads: c_int, kv_heads: c_int, head_dim: c_int,
        max_seq: c_int, scale: f32, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// `qmm_decode_rope_attention` whose launch also loads the first rows of the following one-row GEMV
    /// launches into the L2 of the XCDs that will read them (results unchanged).
    pub fn qmm_decode_rope_attention_warm(
        q: *const f32, k: *const f32, v: *const f32, cos_t: *const f32, sin_t: *const f32, pos: *const i32,
        kcache: *mut f32, vcache: *mut f32, out: *mut f32, heads: c_int, kv_heads: c_int, head_dim: c_int,
        max_seq: c_int, scale: f32, ws: *mut c_void, ws_bytes: usize, warm: *const *const QmmQTensor,
        warm_launch: *const c_int, warm_count: c_int, warm_rows: *const c_int, stream: *mut c_void
    ) -> c_int;

    /// x[i] = table[tokens[first + i]] for i < count (CausalLm embed, llama.rs:397-408);
    /// token ids outside [0, vocab) give NaN rows as in qmm_embed_rows.
    pub fn qmm_embed_rows_n(
        table: *const f32, ld: i64, vocab: i64, tokens: *const i32, first: i64, count: i64, x: *mut f32,
        hidden: i64, stream: *mut c_void
    ) -> c_int;

    /// qmm_rope_kv_append for rows i < count at positions first + i: q and k
    /// rows rotated in place, k and v written to the caches at those positions.
    pub fn qmm_rope_kv_append_n(
        q: *mut f32, k: *mut f32, v: *const f32, ldq: i64, ldk: i64, ldv: i64, cos_t: *const f32,
        sin_t: *const f32, first: i64, count: i64, kcache: *mut f32, vcache: *mut f32, heads: c_int,
        kv_heads: c_int, head_dim: c_int, max_seq: c_int, stream: *mut c_void
    ) -> c_int;

    /// Causal GQA attention of rows i < count: query row i (already rotated, at
    /// position first + i) against cache positions 0 ..= first + i, out row i =
    /// softmax(q . K^T * scale) . V per head (geometry as qmm_decode_attention).
    pub fn qmm_prefill_attention(
        q: *const f32, ldq: i64, kcache: *const f32, vcache: *const f32, first: i64, count: i64,
        out: *mut f32, ldo: i64, heads: c_int, kv_heads: c_int, head_dim: c_int, max_seq: c_int, scale: f32,
        stream: *mut c_void
    ) -> c_int;
    pub fn qmm_prefill_attention_o(
        q: *const f32, ldq: i64, kcache: *const f32, vcache: *const f32, first: i64, count: i64,
        heads: c_int, kv_heads: c_int, head_dim: c_int, max_seq: c_int, scale: f32, wo: *const QmmQTensor,
        x: *mut f32, ldx: i64, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;
    pub fn qmm_prefill_attention_o_workspace_size(wo: *const QmmQTensor, count: i64) -> usize;

    /// h = silu(g) * u over n elements, f32 (LlamaMlp::forward, llama.rs:1386-1391).
    pub fn qmm_silu_mul(g: *const f32, u: *const f32, h: *mut f32, n: i64, stream: *mut c_void) -> c_int;

    /// hq = Q8_K(silu(g) * u) for rows x k (k a multiple of 256), the down
    /// projection's activation (LlamaMlp::forward, llama.rs:1386-1391).
    pub fn qmm_silu_mul_quantize(
        g: *const f32, u: *const f32, rows: i64, k: i64, ld: i64, hq: *mut c_void, stream: *mut c_void
    ) -> c_int;

    /// The down projection of one token with its activation formed in the same
    /// launch: y (+)= QMatMul::forward(silu(g) * u), i.e. qmm_silu_mul_quantize
    /// followed by qmm_matmul_q_ex, with the Q8_K quantization done in the GEMV
    /// prologue (LlamaMlp::forward, llama.rs:1386-1391: down(silu(gate) * up)).
    /// g, u: f32 [w->k] (k-quant weights, k a multiple of 256); y: f32 [w->n];
    /// accumulate != 0 adds to y. Results are identical to the two-call form.
    pub fn qmm_silu_mul_matmul(
        w: *const QmmQTensor, g: *const f32, u: *const f32, y: *mut f32, accumulate: c_int,
        stream: *mut c_void
    ) -> c_int;

    /// Workspace bytes of qmm_greedy_advance; the first 256 bytes are a counter
    /// with the same zero-before-first-use contract as the attention workspace.
    pub fn qmm_greedy_workspace_size(n: i64) -> usize;

    /// Greedy step end on the device: tokens[pos+1] = argmax(logits) (lowest index
    /// on ties, argmax_device, sampler.rs:216-219; a NaN counts as the largest
    /// value, the first NaN wins, as torch.argmax) unless pos+1 < prompt_len (the
    /// slot still holds a prompt token); then pos[0] += 1. `capacity` is the
    /// length of tokens (and of the KV cache): once pos+1 reaches it the call
    /// writes nothing and pos stays, so a step replayed too often never writes
    /// out of bounds.
    pub fn qmm_greedy_advance(
        logits: *const f32, n: i64, tokens: *mut i32, capacity: i64, pos: *mut i32, prompt_len: c_int,
        ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// Routing on the device: logits f32 [tokens, experts] -> softmax -> top-k
    /// (renormalised over the selected experts when `renormalize`). Outputs are
    /// device int32/f32 arrays: counts[experts], offsets[experts + 1] (exclusive
    /// prefix), and tokens*topk (token, weight) pairs grouped by expert in
    /// increasing expert order (pair_token, pair_weight); token_pairs[t*topk + s]
    /// lists token t's pairs in increasing expert order. Replaces the host-side
    /// top-k of llama.rs:1426-1451. Limits: tokens <= 4096, tokens*topk <= 8192.
    pub fn qmm_moe_route(
        logits: *const f32, tokens: i64, experts: c_int, topk: c_int, renormalize: c_int, counts: *mut i32,
        offsets: *mut i32, pair_token: *mut i32, pair_weight: *mut f32, token_pairs: *mut i32,
        stream: *mut c_void
    ) -> c_int;

    /// `qmm_moe_route` with the routed scaling factor (applied when `renormalize` is 0).
    pub fn qmm_moe_route_ex(
        logits: *const f32, tokens: i64, experts: c_int, topk: c_int, renormalize: c_int,
        routed_scaling_factor: f32, counts: *mut i32, offsets: *mut i32, pair_token: *mut i32,
        pair_weight: *mut f32, token_pairs: *mut i32, stream: *mut c_void
    ) -> c_int;

    /// Expert-grouped GEMV (replaces moe_gemm_gguf, ffi.rs:25-39): w[j] (count 1..2)
    /// are stacked expert weights [experts*N, K] of one dtype; xq holds `pairs`
    /// rows of vec-dot blocks grouped by expert (counts/offsets as produced by
    /// qmm_moe_route); y[j] receives [pairs, N] f32. An active expert's weights
    /// are streamed once per 8 of its tokens; experts without tokens read nothing.
    /// Every counts[e] must be <= pairs (the launch is sized for that bound).
    pub fn qmm_moe_gemv(
        w: *const *const QmmQTensor, count: c_int, experts: c_int, xq: *const c_void, pairs: i64,
        counts: *const i32, offsets: *const i32, y: *const *mut f32, stream: *mut c_void
    ) -> c_int;

    /// Expert-grouped prefill GEMM (replaces the grouped prefill launcher
    /// moe/moe_wmma_gguf.cu:124-354 and the per-expert QMatMul::forward over
    /// gathered rows of MoeMlp::forward, llama.rs:1455-1474): x holds `pairs` f32
    /// rows (stride ldx) grouped by expert (counts/offsets as from
    /// qmm_moe_route); y[j] receives [pairs, N] f32 with N = rows / experts. The
    /// rows are quantized once (Q8_K / Q8_0, as QMatMul::forward does), then each
    /// expert's rows go through the int8 MFMA GEMM against its weight slice.
    /// max_rows bounds every count (e.g. the token count for top-k routing).
    /// Outputs equal qmm_matmul's GEMM path on each expert's rows bit for bit.
    /// ws: qmm_moe_gemm_workspace_size(w[0], pairs) bytes; k % 256 == 0.
    pub fn qmm_moe_gemm_workspace_size(w: *const QmmQTensor, pairs: i64) -> usize;

    pub fn qmm_moe_gemm(
        w: *const *const QmmQTensor, count: c_int, experts: c_int, x: *const f32, pairs: i64, ldx: i64,
        max_rows: i64, counts: *const i32, offsets: *const i32, y: *const *mut f32, ws: *mut c_void,
        ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// The whole expert FFN at decode batch sizes: x f32 [tokens, hidden] (row
    /// stride ldx), router logits f32 [tokens, experts], stacked gate/up
    /// [experts*ffn, hidden] and down [experts*hidden, ffn] weights; out f32
    /// [tokens, hidden] (row stride ldo) = sum over each token's top-k experts, in
    /// increasing expert order, of weight * down(silu(gate(x)) * up(x)).
    /// Any token count: a list longer than the routing limit (min(4096, 8192 /
    /// topk) tokens) runs as consecutive chunks of that many tokens, in stream
    /// order through the same workspace; tokens are routed and combined
    /// independently, so the result is the whole list's.
    /// ws: device scratch of qmm_moe_ffn_workspace_size() bytes (one chunk's).
    pub fn qmm_moe_ffn_workspace_size(
        gate: *const QmmQTensor, down: *const QmmQTensor, tokens: i64, experts: c_int, topk: c_int
    ) -> usize;

    pub fn qmm_moe_ffn(
        x: *const f32, tokens: i64, ldx: i64, logits: *const f32, experts: c_int, topk: c_int,
        gate: *const QmmQTensor, up: *const QmmQTensor, down: *const QmmQTensor, out: *mut f32, ldo: i64,
        ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// The whole `MoeMlp::forward`: routed weights renormalised or scaled, and an optional shared
    /// expert (all three weights null: none), gated by sigmoid(x . shared_gate_weight) when that is given.
    pub fn qmm_moe_ffn_ex_workspace_size(
        gate: *const QmmQTensor, down: *const QmmQTensor, tokens: i64, experts: c_int, topk: c_int,
        shared_gate: *const QmmQTensor, shared_up: *const QmmQTensor, shared_down: *const QmmQTensor
    ) -> usize;

    pub fn qmm_moe_ffn_ex(
        x: *const f32, tokens: i64, ldx: i64, logits: *const f32, experts: c_int, topk: c_int,
        norm_topk_prob: c_int, routed_scaling_factor: f32, gate: *const QmmQTensor, up: *const QmmQTensor,
        down: *const QmmQTensor, shared_gate: *const QmmQTensor, shared_up: *const QmmQTensor,
        shared_down: *const QmmQTensor, shared_gate_weight: *const f32, out: *mut f32, ldo: i64,
        ws: *mut c_void, ws_bytes: usize, stream: *mut c_void
    ) -> c_int;

    /// Open a file (memory-mapped, read only) or an in-memory image (copied).
    /// Errors: bad magic, version other than 2 or 3 (QMM_ERR_UNSUPPORTED), counts
    /// above 2^20, truncated tables, tensors of 0 or more than 4 dims, nested
    /// arrays, unknown value types, a data section past the end of the file.
    pub fn qmm_gguf_open(path: *const c_char, out: *mut *mut QmmGguf) -> c_int;

    pub fn qmm_gguf_open_memory(bytes: *const c_void, len: usize, out: *mut *mut QmmGguf) -> c_int;

    pub fn qmm_gguf_close(g: *mut QmmGguf);

    pub fn qmm_gguf_version(g: *const QmmGguf) -> c_int;

    /// general.alignment when it is an integer (>= 1), else 32.
    pub fn qmm_gguf_alignment(g: *const QmmGguf) -> u64;

    pub fn qmm_gguf_tensor_count(g: *const QmmGguf) -> i64;

    pub fn qmm_gguf_metadata_count(g: *const QmmGguf) -> i64;

    /// Index of a tensor / metadata key (-1 if absent; a repeated key keeps its last value).
    pub fn qmm_gguf_find_tensor(g: *const QmmGguf, name: *const c_char) -> i64;

    pub fn qmm_gguf_meta_find(g: *const QmmGguf, key: *const c_char) -> i64;

    /// Tensor i: name (owned by g), dims, shape in torch order (the GGML ne order
    /// reversed: [out, in] for a linear weight; unused entries 0), GGML type tag
    /// and byte offset within the data section.
    pub fn qmm_gguf_tensor_info(
        g: *const QmmGguf, i: i64, name: *mut *const c_char, ndims: *mut c_int, shape: *mut i64,
        ggml_type: *mut c_int, offset: *mut u64
    ) -> c_int;

    /// (elements, bytes) per block of a GGML type tag (dequant.rs:86-140).
    pub fn qmm_gguf_type_size(ggml_type: c_int, block_elems: *mut u64, block_bytes: *mut u64) -> c_int;

    /// Host pointer to tensor i's bytes inside the file and their length
    /// (elements / block_elems * block_bytes); out-of-range data is an error.
    pub fn qmm_gguf_tensor_data(
        g: *const QmmGguf, i: i64, data: *mut *const c_void, bytes: *mut usize
    ) -> c_int;

    /// Metadata entry i: key, value type (GGUF tags 0..12; 9 = array), element
    /// type (arrays) and count (1 for scalars). Values: elem = -1 for a scalar,
    /// else the array element. u64 takes unsigned integers, non-negative signed
    /// ones and bools; i64 any integer; f64 f32/f64; string a pointer into the
    /// file (not NUL-terminated) and its length. A type mismatch is an error.
    pub fn qmm_gguf_meta_info(
        g: *const QmmGguf, i: i64, key: *mut *const c_char, type_: *mut c_int, elem_type: *mut c_int,
        count: *mut u64
    ) -> c_int;

    pub fn qmm_gguf_meta_u64(g: *const QmmGguf, i: i64, elem: i64, v: *mut u64) -> c_int;

    pub fn qmm_gguf_meta_i64(g: *const QmmGguf, i: i64, elem: i64, v: *mut i64) -> c_int;

    pub fn qmm_gguf_meta_f64(g: *const QmmGguf, i: i64, elem: i64, v: *mut f64) -> c_int;

    pub fn qmm_gguf_meta_string(
        g: *const QmmGguf, i: i64, elem: i64, s: *mut *const c_char, len: *mut u64
    ) -> c_int;

    /// Resident load of a 2-D Q8_0 / Q4_K / Q6_K tensor into a device QTensor
    /// (QStorage::from_data + QTensor::new, candle-gen/src/quant/repack.rs:202-203),
    /// on the current device, synchronous. unpermute_heads > 0 undoes llama.cpp's
    /// q/k row order per head on the quantized rows (unpermute_qk, candle-llm
    /// gguf.rs:333-356: torch row k * hd/2 + j of a head is GGUF row 2j + k).
    pub fn qmm_gguf_load_qtensor(
        g: *const QmmGguf, i: i64, unpermute_heads: c_int, stream: *mut c_void, out: *mut *mut QmmQTensor
    ) -> c_int;

    /// Measurement aid, no counterpart in the reference: a plain streaming read
    /// of `bytes` (a multiple of 16) at `data` on the device, the ceiling a
    /// weight-streaming launch of the same size is measured against. variant:
    /// 0 grid-stride with 4 loads in flight per thread, 1 grid-stride with 8,
    /// 2 one contiguous chunk per workgroup with 8 nontemporal loads in flight
    /// (no variant is fastest at every size). wgs_per_cu workgroups of 256
    /// threads per CU (0: 8; at most 64); `sink` (one word) is written only if
    /// the folded data equals a fixed constant.
    pub fn qmm_stream_read(
        data: *const c_void, bytes: usize, sink: *mut u32, variant: c_int, wgs_per_cu: c_int,
        stream: *mut c_void
    ) -> c_int;
}

// ---------------------------------------------------------------------------
// Safe layer: the calls the engine's QTensor / QMatMul path makes.
// ---------------------------------------------------------------------------

/// A failed call: the status and the library's message for this thread.
#[derive(Debug, Clone)]
pub struct QmmError {
    pub status: c_int,
    pub message: String,
}

impl std::fmt::Display for QmmError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "qmm error {}: {}", self.status, self.message)
    }
}

impl std::error::Error for QmmError {}

/// Maps a status to `Ok` or the thread's last error message.
pub fn check(status: c_int) -> Result<(), QmmError> {
    if status == QMM_OK {
        return Ok(());
    }
    let message = unsafe { CStr::from_ptr(qmm_last_error()) }.to_string_lossy().into_owned();
    Err(QmmError { status, message })
}

/// A block-quantized [n, k] weight resident on one GPU (candle's `QTensor` on this backend).
pub struct QTensor {
    raw: *mut QmmQTensor,
}

unsafe impl Send for QTensor {}

impl QTensor {
    /// `QStorage::from_data` of GGML block bytes held on the host. `bytes` must hold exactly the
    /// tensor's n * (k / block) blocks: the C side copies that many bytes from it, so a slice of any
    /// other length is refused here (QMM_ERR_INVALID) before the call.
    pub fn from_ggml(dtype: c_int, n: i64, k: i64, bytes: &[u8], stream: *mut c_void) -> Result<Self, QmmError> {
        let invalid = |what: &str| QmmError { status: QMM_ERR_INVALID, message: what.to_string() };
        let (bs, ts) = unsafe { (qmm_block_size(dtype), qmm_type_size(dtype)) };
        if bs <= 0 || ts <= 0 {
            return Err(invalid("unsupported dtype"));
        }
        if n <= 0 || k <= 0 || k % bs as i64 != 0 {
            return Err(invalid("shape is empty or k is not a whole number of blocks"));
        }
        let want = (n as u64)
            .checked_mul((k / bs as i64) as u64)
            .and_then(|blocks| blocks.checked_mul(ts as u64))
            .ok_or_else(|| invalid("tensor byte count overflows"))?;
        if bytes.len() as u64 != want {
            return Err(invalid("byte slice length differs from the tensor's GGML byte count"));
        }
        let mut raw = std::ptr::null_mut();
        check(unsafe {
            qmm_qtensor_from_ggml(dtype, n, k, bytes.as_ptr() as *const c_void, 0, stream, &mut raw)
        })?;
        Ok(QTensor { raw })
    }

    /// `QTensor::quantize` of a dense f32 [n, k] weight already on the device.
    pub fn quantize(dtype: c_int, n: i64, k: i64, w_dev: *const f32, stream: *mut c_void) -> Result<Self, QmmError> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { qmm_qtensor_quantize(dtype, n, k, w_dev, stream, &mut raw) })?;
        Ok(QTensor { raw })
    }

    /// (dtype, n, k).
    pub fn info(&self) -> Result<(c_int, i64, i64), QmmError> {
        let (mut dt, mut n, mut k) = (0, 0, 0);
        check(unsafe { qmm_qtensor_info(self.raw, &mut dt, &mut n, &mut k) })?;
        Ok((dt, n, k))
    }

    pub fn as_raw(&self) -> *const QmmQTensor {
        self.raw
    }

    /// Workspace bytes `matmul` needs for `m` activation rows.
    pub fn matmul_workspace_size(&self, m: i64) -> usize {
        unsafe { qmm_matmul_workspace_size(self.raw, m) }
    }

    /// `QMatMul::forward`: y[m, n] = x[m, k] . W^T, x and y f32 on the device, `ws` a device buffer of
    /// `matmul_workspace_size(m)` bytes owned by the caller (one per concurrent stream).
    pub unsafe fn matmul(
        &self, x: *const f32, m: i64, ldx: i64, y: *mut f32, ldy: i64, ws: *mut c_void, ws_bytes: usize,
        stream: *mut c_void,
    ) -> Result<(), QmmError> {
        check(qmm_matmul(self.raw, x, m, ldx, y, ldy, ws, ws_bytes, stream))
    }

    /// `QTensor::dequantize` into a dense f32 [n, k] device buffer.
    pub unsafe fn dequantize(&self, dst: *mut f32, stream: *mut c_void) -> Result<(), QmmError> {
        check(qmm_qtensor_dequantize(self.raw, dst, stream))
    }
}

impl Drop for QTensor {
    fn drop(&mut self) {
        unsafe { qmm_qtensor_free(self.raw) }
    }
}

/// A GGUF file opened by the library's parser (`gguf_file::Content::read`).
pub struct Gguf {
    raw: *mut QmmGguf,
}

impl Gguf {
    pub fn open(path: &str) -> Result<Self, QmmError> {
        let c = CString::new(path).map_err(|_| QmmError { status: QMM_ERR_INVALID, message: "path".into() })?;
        let mut raw = std::ptr::null_mut();
        check(unsafe { qmm_gguf_open(c.as_ptr(), &mut raw) })?;
        Ok(Gguf { raw })
    }

    /// `Content::tensor(...)` of a quantized 2-D tensor straight into a device QTensor (q/k rows
    /// un-permuted from llama.cpp's order when `unpermute_heads` > 0).
    pub fn load_qtensor(&self, name: &str, unpermute_heads: c_int, stream: *mut c_void) -> Result<QTensor, QmmError> {
        let c = CString::new(name).map_err(|_| QmmError { status: QMM_ERR_INVALID, message: "name".into() })?;
        let i = unsafe { qmm_gguf_find_tensor(self.raw, c.as_ptr()) };
        if i < 0 {
            return Err(QmmError { status: QMM_ERR_INVALID, message: format!("no tensor {name}") });
        }
        let mut raw = std::ptr::null_mut();
        check(unsafe { qmm_gguf_load_qtensor(self.raw, i, unpermute_heads, stream, &mut raw) })?;
        Ok(QTensor { raw })
    }
}

impl Drop for Gguf {
    fn drop(&mut self) {
        unsafe { qmm_gguf_close(self.raw) }
    }
}

/*
 * ggml_mi355x_kernels.h -- C ABI of the MI355X (gfx950) decode kernels.
 *
 * This layer replaces the reference's aclnn operator ABI (two-phase
 * aclnnXxxGetWorkspaceSize + aclnnXxx(ws, n, exec, stream)) that the CANN
 * backend calls on the decode hot path.  Every entry point takes plain device
 * pointers, sizes and a hipStream_t passed as void*, returns 0 on success or a
 * negative MI_ERR_* / positive hipError_t code, never aborts, and keeps no
 * global state other than per-device lazily created function handles and the
 * fixed per-device scratch array of mi_fa_decode_noalloc.
 * The last error message of the calling thread is available from
 * mi_last_error().
 *
 * Reference citations are relative to the reference repository
 * (patch:N = line N of patches/ascend310b4-llama-cpp.patch).
 */
#ifndef GGML_MI355X_KERNELS_H
#define GGML_MI355X_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_OK            0
#define MI_ERR_ARG      -1   /* bad size / shape / null pointer */
#define MI_ERR_ALIGN    -2   /* pointer or stride alignment not supported */
#define MI_ERR_WORKSPACE -3  /* workspace too small */
#define MI_ERR_NODEVICE -4   /* no HIP device */
#define MI_ERR_UNSUPPORTED -5

/* activation quantizer rounding (ggml-CPU has two): */
#define MI_Q8_ROUND_REF 0    /* ggml quantize_row_q8_0_ref: id = 1/d, round half away from zero */
#define MI_Q8_ROUND_X86 1    /* ggml-cpu x86 SIMD quantize_row_q8_0: id = 127/amax, round half to even */

const char *mi_last_error(void);

/* ------------------------------------------------------------------------
 * Device plumbing used by hosts that have no other HIP runtime (tests,
 * benchmarks, the ggml adapter).  Thin wrappers of hipMalloc & co.
 * ---------------------------------------------------------------------- */
int mi_device_count(int *count);
int mi_set_device(int device);
int mi_device_name(int device, char *buf, size_t len);
int mi_malloc(void **ptr, size_t bytes);
int mi_free(void *ptr);
int mi_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int mi_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int mi_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
int mi_memset(void *dst, int value, size_t bytes, void *stream);
int mi_stream_create(void **stream);
int mi_stream_destroy(void *stream);
int mi_stream_sync(void *stream);
int mi_device_sync(void);
int mi_event_create(void **event);
int mi_event_destroy(void *event);
int mi_event_record(void *event, void *stream);
int mi_event_elapsed_ms(float *ms, void *start, void *stop);
/* stream capture into a HIP graph (launch-overhead-free replay of a fixed launch sequence);
 * nothing captured may call hipMemsetAsync */
int mi_graph_capture_begin(void *stream);
int mi_graph_capture_end(void *stream, void **graph_exec);
int mi_graph_launch(void *graph_exec, void *stream);
int mi_graph_destroy(void *graph_exec);

/* ------------------------------------------------------------------------
 * Weight prepack (replaces the set_tensor side layouts: FRACTAL_NZ via
 * aclnnTransMatmulWeight patch:1700-1809, and the host A8W8 transform
 * ggml_backend_cann_transform_f16_a8w8 patch:1674-1695; sizes replace
 * ggml_cann_310b_nz_size / a8w8_size patch:1535-1562).
 *
 * Q8_0 packed layout for a weight of n rows x k columns (nb = k/32 blocks
 * per row), three 256-byte-aligned planes:
 *   qlo [n][nb][16] int8   -- qs[0..15]  of block (row, b)
 *   qhi [n][nb][16] int8   -- qs[16..31] of block (row, b)
 *   d   [n][nb]     fp16   -- block scale
 * Q4_0 packed layout: qs [n][nb][16] (ggml nibble order kept), d [n][nb] fp16.
 * src is ggml block_q8_0 / block_q4_0 rows (34 / 18 bytes per block).
 * ---------------------------------------------------------------------- */
size_t mi_q8_0_packed_size(int64_t n, int64_t k);
size_t mi_q4_0_packed_size(int64_t n, int64_t k);
int mi_prepack_q8_0(void *stream, const void *src_blocks, void *dst_packed, int64_t n, int64_t k);
int mi_prepack_q4_0(void *stream, const void *src_blocks, void *dst_packed, int64_t n, int64_t k);
/* host-side versions of the same layouts (byte-identical to the device ones) */
int mi_prepack_q8_0_host(const void *src_blocks, void *dst_packed, int64_t n, int64_t k);
int mi_prepack_q4_0_host(const void *src_blocks, void *dst_packed, int64_t n, int64_t k);
int mi_unpack_q8_0_host(const void *packed, void *dst_blocks, int64_t n, int64_t k);
int mi_unpack_q4_0_host(const void *packed, void *dst_blocks, int64_t n, int64_t k);
/* A8W8 weight quantization at upload (replaces ggml_backend_cann_transform_f16_a8w8,
 * patch:1674-1695, run by set_tensor at patch:1716-1751 for the weights
 * ggml_cann_310b_is_a8w8_weight selects, patch:1520-1533).  An F16 weight [n][k] (ggml
 * rows, k contiguous) times the SmoothQuant factors s[k] (fp32, NULL = none) is quantized
 * per 32-block to Q8_0 with quantize_row_q8_0_ref's rounding (d = amax/127 stored fp16,
 * q = round-half-away(v/d)) and written in the Q8_0 packed layout above.  The reference
 * quantizes per output channel into FRACTAL_NZ int8; here the A8W8 weight format is ggml
 * Q8_0, so the same GEMVs serve quantized GGUFs and F16 GGUFs quantized at load.
 * w_f16 8-byte aligned, s 16-byte aligned, dst 256-byte aligned. */
int mi_quantize_f16_q8_0(void *stream, const uint16_t *w_f16, const float *s, void *dst_packed, int64_t n,
                         int64_t k);

/* ------------------------------------------------------------------------
 * Activation quantization (replaces aclnnW8a8QuantizeCustom,
 * experiments/a8w8/w8a8_quantize_custom_vector.cpp:97-106, plus the fp32->fp16
 * cast before it, patch:1266-1267).  ggml Q8_0 per 32-block semantics.
 * x     : fp32 [m][k]
 * inv_s : fp32 [k] SmoothQuant reciprocal factors (x*inv_s is quantized), or NULL
 * xq    : output, planar: qs int8 [m][k] at xq, d fp16 [m][k/32] at xq + mi_xq_d_offset(m,k)
 * ---------------------------------------------------------------------- */
size_t mi_xq_size(int64_t m, int64_t k);
size_t mi_xq_d_offset(int64_t m, int64_t k);
int mi_act_quant_q8_0(void *stream, const float *x, const float *inv_s, int64_t m, int64_t k, void *xq,
                      int rounding);

/* ------------------------------------------------------------------------
 * A8W8 Q8_0 GEMV, m <= 8 activation rows (replaces aclnnMatmulW8a8I32Custom +
 * W8a8DequantCustom + cast, patch:1268-1271; kernel
 * experiments/a8w8/custom_ops_nz/op_kernel/matmul_w8a8_i32_custom.cpp:15-48).
 * y[i][row] = sum_b float(sumi(row,b,i)) * (d_w(row,b) * d_x(i,b)), sumi exact int32.
 * ---------------------------------------------------------------------- */
int mi_gemv_q8_0(void *stream, const void *w_packed, const void *xq, float *y, int64_t n, int64_t k,
                 int64_t m);
/* the whole A8W8 branch of ggml_cann_mat_mul_fp (patch:1223-1281): quantize x (with
 * optional inv_s) then GEMV.  For m == 1 and k <= 4096 the quantization runs in the GEMV
 * prologue (one launch, no workspace); otherwise ws must hold
 * mi_mul_mat_q8_0_workspace_size(m, k) bytes for the quantized activation. */
size_t mi_mul_mat_q8_0_workspace_size(int64_t m, int64_t k);
int mi_mul_mat_q8_0_f32(void *stream, const void *w_packed, const float *x, const float *inv_s, float *y,
                        int64_t n, int64_t k, int64_t m, int rounding, void *ws, size_t ws_bytes);
/* the same for up to four matrices of equal k that read one activation row (q/k/v or
 * gate/up): rows of matrix i go to y[i]; a single launch when k <= 4096, otherwise one
 * quantization into ws and one GEMV per matrix */
int mi_mul_mat_q8_0_f32_multi(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, int64_t k, const float *x, const float *inv_s, int rounding, void *ws,
                              size_t ws_bytes);
/* ------------------------------------------------------------------------
 * The decoder layers of one A8W8 decode token as ONE persistent launch (the
 * backend's whole-layer-stack fusion).  Replaces, for a run of consecutive layers,
 * the reference's node-by-node evaluation (evaluate_and_capture_cann_graph,
 * patch:1897-1930) of RMS_NORM, MUL, MUL_MAT (q/k/v/o/gate/up/down, Q8_0 A8W8 with
 * SmoothQuant), ADD, ROPE, SET_ROWS, FLASH_ATTN_EXT (patch:1370-1432), GLU.
 * A grid of one resident workgroup per CU walks every layer through five phases
 * (q/k/v + RoPE + KV write; attention splits; split merge + o + residual; RMSNorm +
 * gate/up + swiglu; quantization + down + residual) separated by in-kernel dependency
 * hops; results are bit-identical to the per-node launches.  Shapes: Qwen2.5-1.5B-like
 * (n_embd 1536, head_dim 128, 6 q heads per kv head, n_ff 8960), one sequence, an
 * attention view of at most 1024 positions (16 splits), 256 CUs.
 * ---------------------------------------------------------------------- */
typedef struct mi_persist_layer {
    const void *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down; /* Q8_0 packed (mi_prepack_q8_0 layout) */
    const float *bq, *bk, *bv;                              /* q/k/v biases, or NULL */
    const float *attn_norm, *ffn_norm;                      /* RMSNorm weights [n_embd] */
    const float *inv_s_attn, *inv_s_o, *inv_s_ffn, *inv_s_down; /* SmoothQuant 1/s of each input, or NULL */
    void *k_cache, *v_cache;  /* fp16 [n_cache_rows][n_head_kv*head_dim]; row kv_idx is written */
} mi_persist_layer;

typedef struct mi_persist_args {
    const float *x_in;         /* the first layer's input (residual stream) fp32 [n_embd] */
    float *x_out;              /* the last layer's output fp32 [n_embd]; the layers in between
                                  keep theirs in the context's scratch */
    const int32_t *pos;        /* RoPE position (device, 1 value) */
    const void *kv_idx;        /* cache row to write (device, 1 value, int32 or int64) */
    int kv_idx_is_i64;
    int64_t n_cache_rows;
    size_t kv_row_bytes;       /* K and V cache row stride */
    int n_kv;                  /* attention view length (positions) */
    const int32_t *kv_len;     /* effective length (the FLASH_ATTN_EXT src[5]), or NULL */
    const uint16_t *mask;      /* F16 KQ mask over the view (the FLASH_ATTN_EXT src[3], one row of
                                  >= n_kv elements, added to the scaled scores), or NULL */
    float kq_scale, rms_eps;
    float freq_base, freq_scale, attn_factor;  /* neox RoPE over the head dim */
    int rounding;              /* MI_Q8_ROUND_* of the activation quantizations */
    long spin_limit;           /* polls before a dependency wait gives up (<= 0: default, seconds) */
    int debug_stall_hop;       /* -1; h in 0..4: the waits on hop h of the first layer expect one
                                  arrival more than its producers make, so they give up after
                                  spin_limit polls (tests of the error path) */
    const uint16_t *embd;      /* or, with x_in NULL: the first layer's input is row tok[0] of this
                                  F16 table (the token embedding; GET_ROWS folded in), rows embd_ld
                                  elements apart, 8-byte aligned */
    int64_t embd_ld;
    const int32_t *tok;        /* the row index (device, 1 value) */
} mi_persist_args;

/* context: scratch (per-layer intermediates), counters, pinned error word; allocates */
int mi_persist_create(void **ctx, int device, int n_layer, int n_embd, int n_head, int n_head_kv, int head_dim,
                      int n_ff);
void mi_persist_destroy(void *ctx);
/* the layers' tensors (host array).  When it differs from the last call's it is copied
 * to the device after the stream synchronised (a launch in flight may still read the
 * old one): call outside stream capture; an unchanged array does nothing. */
int mi_persist_set_layers(void *stream, void *ctx, const mi_persist_layer *layers, int n_layer);
/* 1 when the pipeline is instantiated for this shape and an attention view of n_kv
 * positions fits its split records (at most 16 splits), else 0 */
int mi_persist_supported(int64_t n_kv, int n_embd, int n_head, int n_head_kv, int head_dim, int n_ff);
/* one launch over all layers (no allocation, capturable) */
int mi_persist_decode_q8_0(void *stream, void *ctx, const mi_persist_args *args);
/* phase timestamps (profiling): after enable_trace (allocates), every launch records the
 * device wall clock at its phase boundaries per layer and workgroup; read_trace copies the
 * last launch's [n_layer][n_wg][n_events] words (dst NULL: only the sizes and the clock
 * rate in ticks per microsecond) */
int mi_persist_enable_trace(void *ctx);
int mi_persist_read_trace(void *ctx, uint64_t *dst, size_t n_words, int *n_layer, int *n_wg, int *n_events,
                          double *ticks_per_us);
/* after the stream synchronised: MI_OK, or an error when a dependency wait gave up in a
 * launch since the last call (that launch's results are invalid) */
int mi_persist_status(void *ctx);

/* ---- fused decode chains (the backend's graph fusions).  Each replaces a run of
 * adjacent ggml nodes of llama.cpp's decode graph with one launch; the reference's
 * evaluate_and_capture_cann_graph runs every node through ggml_cann_compute_forward
 * one by one (patch:1897-1930). ---- */

/* [RMS_NORM -> MUL(norm_w)] -> MUL_MAT x n_mats (Q8_0, one activation row, k <= 4096;
 * without a norm k <= 12288, e.g. the down projection of a gate/up pair)
 * -> optional ADD of add[i] (bias or residual, length n[i]) per matrix.  norm_w == NULL
 * skips the RMSNorm (x is the activation itself). */
int mi_mul_mat_q8_0_f32_fused(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *add, int64_t k, const float *x,
                              const float *norm_w, float eps, const float *inv_s, int rounding);
/* A ubatch (m = 2..8 activation rows) through up to four Q8_0 matrices of equal k that
 * read the same activation, in two launches: the activation rows' Q8_0 blocks with
 * their producer folded in (RMSNorm(x) * norm_w when norm_w is set, k <= 4096; else
 * silu(x) * x_up when x_up is set, ggml's swiglu; else x), times inv_s; then one GEMV
 * launch over the stacked matrices with the blocks staged in LDS.  Matrix i writes
 * y[i] [m, n[i]] (row-major, ggml's MUL_MAT layout) plus bias[i] (a row of n[i],
 * broadcast) or add[i] ([m, n[i]], a residual), either may be NULL.  Bit-identical to
 * RMS_NORM + MUL (or GLU) then mi_mul_mat_q8_0_f32 per matrix then ADD.  ws:
 * mi_xq_size(m, k) bytes, 16-byte aligned.  Cf. the reference's M <= 8 matmul
 * routing (patch:1207, 1286-1309): one kernel per projection there. */
int mi_mul_mat_q8_0_f32_batch(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *bias, const float *const *add, int64_t k, int64_t m,
                              const float *x, const float *x_up, const float *norm_w, float eps, const float *inv_s,
                              int rounding, void *ws, size_t ws_bytes);
/* FLASH_ATTN_EXT (one token, one sequence) -> MUL_MAT(Q8_0) [-> ADD(add)]: the projection
 * of an attention output left in split form by mi_fa_decode_partials.  Every workgroup
 * merges the n_splits records (the log-sum-exp combine of mi_fa_decode) for its whole
 * activation row in its prologue, so no combine launch and no attention-output tensor.
 * k = n_heads * head_dim <= 2048, n_splits <= 16, head_dim % 4 == 0; add may be NULL.
 * Replaces the reference's attention output handed to the o projection
 * (patch:1370-1432, then ggml_cann_mat_mul_fp patch:1188-1355). */
int mi_mul_mat_q8_0_f32_lse(void *stream, const void *w_packed, int64_t n, float *y, const float *add,
                            const float *part, int64_t n_splits, int64_t n_heads, int64_t head_dim,
                            const float *inv_s, int rounding);
/* Several activation rows (m in 1..16: the tokens of one ubatch, e.g. one per sequence) through
 * n_mats Q4_0 MUL_MATs of equal k that read the same activation (q/k/v, gate/up), in one launch
 * after one fp16 conversion of the activation: y[i] = W_i x (+ bias[i] broadcast over the rows)
 * (+ add[i], a full [m][n[i]] tensor: the residual), each optional (bias / add or their entries
 * may be NULL).  x: fp32 [m][k]; with up != NULL the activation is ggml swiglu(x, up) =
 * x / (1 + expf(-x)) * up (the GLU node before the down projection); with norm_w != NULL it
 * is RMS_NORM(x, eps) * norm_w per row (k <= 4096, x and norm_w 16-byte aligned); up and
 * norm_w exclusive.  k % 128 == 0; ws of m*k*2 bytes, 16-byte aligned.  Replaces, per
 * matrix, the ggml_cann_mat_mul_fp route for a batch of rows (patch:1207) and the
 * RMS_NORM / MUL / ADD / GLU nodes around it. */
int mi_mul_mat_q4_0_f32_batch(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *bias, const float *const *add, int64_t k,
                              int64_t m, const float *x, const float *up, const float *norm_w, float eps, void *ws,
                              size_t ws_bytes);
/* The same projections from an activation already converted: xp holds the m rows as fp16,
 * each 32-element block permuted as xp[row][block][g][8] = x[4g], x[4g+2], x[4g+1],
 * x[4g+3], x[16+4g], x[18+4g], x[17+4g], x[19+4g] (g = 0..3), 16-byte aligned, as
 * mi_fa_decode_batch_q4act writes the attention output.  No reference counterpart: the
 * reference runs one row per projection (patch:1207). */
int mi_mul_mat_q4_0_batch_xp(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                             float *const *y, const float *const *bias, const float *const *add, int64_t k,
                             int64_t m, const void *xp);
/* [RMS_NORM -> MUL(norm_w)] -> gate and up MUL_MATs (Q4_0, n x k each) -> GLU swiglu for
 * m activation rows (1..16) in two launches: hxp gets fp16(silu(gate) * up) as the down
 * projection's activation in mi_mul_mat_q4_0_batch_xp's permuted layout (m * n * 2 bytes,
 * 16-byte aligned), bit-identical to mi_mul_mat_q4_0_f32_batch of the gate/up pair followed
 * by that call's GLU conversion.  k % 128 == 0, n % 128 == 0; ws: m * k * 2 bytes, not
 * overlapping hxp.  No reference counterpart: the reference runs one row per matmul and
 * the SwiGLU node apart (patch:1207). */
int mi_mul_mat_q4_0_gate_up_glu_batch(void *stream, const void *w_gate, const void *w_up, int64_t n, int64_t k,
                                      int64_t m, const float *x, const float *norm_w, float eps, void *ws,
                                      size_t ws_bytes, void *hxp);
/* [RMS_NORM -> MUL(norm_w)] -> q/k/v MUL_MATs (Q4_0, w_packed[0..2], n[0..2] rows) ->
 * ADD bias[i] (or NULL) -> neox ROPE of q and k (position pos[r] for activation row r,
 * head_dim rows per head) -> SET_ROWS of k and v (fp16) into cache row kv_idx[r], for m
 * activation rows (1..16) in two launches; q_out gets the rotated q ([m][n[0]] fp32).
 * Bit-identical to mi_mul_mat_q4_0_f32_batch of the set (with the biases) followed by
 * mi_rope_kv_rows.  head_dim a multiple of 32 up to 256, n[0] and n[1] multiples of it,
 * n[2] of 32, k % 128 == 0; ws: m * k * 2 bytes.  No reference counterpart: the
 * reference runs these nodes one row and one node at a time. */
int mi_qkv_rope_kv_q4_0_batch(void *stream, const void *const *w_packed, const int64_t *n, const float *const *bias,
                              int64_t k, int64_t m, const float *x, const float *norm_w, float eps, void *ws,
                              size_t ws_bytes, int64_t head_dim, const int32_t *pos, float freq_base,
                              float freq_scale, float attn_factor, float *q_out, void *k_cache, size_t k_row_bytes,
                              void *v_cache, size_t v_row_bytes, const void *kv_idx, int kv_idx_is_i64,
                              int64_t n_cache_rows);
/* the attention-input chain of one token: [RMS_NORM -> MUL(norm_w)] -> q/k/v MUL_MATs
 * (w_packed[0..2], n[0..2] rows, k <= 4096) -> ADD bias[i] (or NULL) -> neox ROPE of q
 * and k (n_dims = head_dim, theta = pos[0] * freq_base^(-2i/head_dim), freq_scale,
 * attn_factor; ext_factor 0) -> q fp32 into q_out[n[0]], k and v converted to fp16 into
 * row kv_idx[0] (int32, or int64 when kv_idx_is_i64) of the caches (SET_ROWS); rows
 * outside [0, n_cache_rows) are not written.  rope_table: mi_rope_table's output for
 * pos[0] and the same parameters, or NULL to form the angles in the launch. */
int mi_qkv_rope_kv_q8_0(void *stream, const void *const *w_packed, const int64_t *n, const float *const *bias,
                        int64_t k, const float *x, const float *norm_w, float eps, const float *inv_s, int rounding,
                        int64_t head_dim, const int32_t *pos, float freq_base, float freq_scale, float attn_factor,
                        float *q_out, void *k_cache, size_t k_row_bytes, void *v_cache, size_t v_row_bytes,
                        const void *kv_idx, int kv_idx_is_i64, int64_t n_cache_rows, const float *rope_table);
/* [RMS_NORM -> MUL(norm_w)] -> gate and up MUL_MATs (Q8_0, n_ff x k each, one activation
 * row, k <= 2048, SmoothQuant inv_s of both) -> GLU swiglu -> the down projection's Q8_0
 * activation quantization (its SmoothQuant inv_s_down, length n_ff, or NULL) in one
 * launch: xq as mi_act_quant_q8_0 writes it for (1, n_ff), ready for mi_gemv_q8_0_add.
 * n_ff % 32 == 0.  Bit-identical to mi_mul_mat_q8_0_f32_fused then mi_swiglu_quant_q8_0.
 * Replaces the CANN gate/up matmuls and the SwiGLU node before the down projection
 * (patch:1188-1355 per matmul). */
int mi_gate_up_swiglu_q8_0(void *stream, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k,
                           const float *x, const float *norm_w, float eps, const float *inv_s,
                           const float *inv_s_down, int rounding, void *xq);
/* [RMS_NORM -> MUL(norm_w)] -> gate and up MUL_MATs (Q8_0, n_ff x k each, one activation
 * row, k <= 2048, SmoothQuant inv_s of both) -> GLU swiglu times inv_s_down (length n_ff,
 * or NULL): h fp32 [n_ff], the down projection's input before its Q8_0 quantization, which
 * mi_mul_mat_q8_0_f32_fused (norm_w and inv_s NULL, n_ff <= 12288) does in its prologue.
 * A workgroup pairs 8 gate rows with the same 8 up rows: n_ff % 8 == 0.  h and its
 * quantization are bit-identical to mi_mul_mat_q8_0_f32_fused then mi_swiglu_quant_q8_0.
 * Replaces the CANN gate/up matmuls and the SwiGLU node before the down projection
 * (patch:1188-1355 per matmul). */
int mi_gate_up_swiglu_f32_q8_0(void *stream, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k,
                               const float *x, const float *norm_w, float eps, const float *inv_s,
                               const float *inv_s_down, int rounding, float *h);
/* mi_gate_up_swiglu_q8_0's result (xq of the swiglu times inv_s_down, ready for
 * mi_gemv_q8_0_add) from the grid of mi_gate_up_swiglu_f32_q8_0: a workgroup pairs 8 gate
 * rows with the same 8 up rows, and the last of the four workgroups of each 32-block
 * (counted on counters[block]) quantizes the block.  h_tmp: n_ff floats (16-byte
 * aligned) for the swiglu values; counters: n_ff / 32 words, zero before the first call,
 * left zero by every call.  n_ff % 32 == 0, k <= 2048.  Calls that overlap on the same
 * counters race.  Bit-identical to mi_mul_mat_q8_0_f32_fused then mi_swiglu_quant_q8_0.
 * Replaces the CANN gate/up matmuls and the SwiGLU node (patch:1188-1355 per matmul). */
int mi_gate_up_pair_q8_0(void *stream, const void *w_gate, const void *w_up, int64_t n_ff, int64_t k, const float *x,
                         const float *norm_w, float eps, const float *inv_s, const float *inv_s_down, int rounding,
                         void *xq, float *h_tmp, unsigned *counters);
/* GLU swiglu(g, u) of one row (k floats) times inv_s, quantized to Q8_0 into xq (the
 * planar layout of mi_act_quant_q8_0 with m = 1): the input side of the down projection */
int mi_swiglu_quant_q8_0(void *stream, const float *g, const float *u, const float *inv_s, int64_t k, void *xq,
                         int rounding);
/* mi_gemv_q8_0 with the ADD of a same-shape vector (residual) fused: y = W*xq + add */
int mi_gemv_q8_0_add(void *stream, const void *w_packed, const void *xq, const float *add, float *y, int64_t n,
                     int64_t k, int64_t m);

/* debug: exact per-block int32 dot products out[row][b] for activation row 0 */
int mi_q8_0_block_dots(void *stream, const void *w_packed, const void *xq, int32_t *out, int64_t n, int64_t k);

/* ------------------------------------------------------------------------
 * W4A16 GEMV, int4 group-32 (ggml Q4_0) x fp16 activations, fp32 accumulation
 * (replaces the add-on's standalone add_custom operator,
 * experiments/w4a16-gemv/source/w4a16_gemv_qwen.cpp:24-180).
 * x_f16 : fp16 [m][k];  y : fp32 [m][n]
 * ---------------------------------------------------------------------- */
int mi_gemv_q4_0_f16(void *stream, const void *w_packed, const uint16_t *x_f16, float *y, int64_t n, int64_t k,
                     int64_t m);
/* the same with the ADD of a same-shape vector (residual) fused: y = W*x + add */
int mi_gemv_q4_0_f16_add(void *stream, const void *w_packed, const uint16_t *x_f16, const float *add, float *y,
                         int64_t n, int64_t k, int64_t m);
/* W4A16 decode chains, one activation row (m = 1, k <= 4096; without the norm the
 * first one takes k <= 32256), the counterparts of the
 * Q8_0 chains above (node sequences of the Qwen2 graph builder, per-node dispatch
 * patch:1897-1930 in the reference):
 * [RMS_NORM -> MUL(norm_w)] -> n_mats MUL_MATs sharing src1 (stacked rows) -> ADD add[i]
 * (residual or bias, or NULL) */
int mi_mul_mat_q4_0_f32_fused(void *stream, int n_mats, const void *const *w_packed, const int64_t *n,
                              float *const *y, const float *const *add, int64_t k, const float *x,
                              const float *norm_w, float eps);
/* [RMS_NORM -> MUL(norm_w)] -> gate and up MUL_MATs (n rows each) -> GLU swiglu
 * (silu(gate) * up) -> fp16 h_out[n] (RNE, the conversion the down projection's MUL_MAT
 * applies to its src1) */
int mi_gate_up_swiglu_q4_0(void *stream, const void *w_gate, const void *w_up, int64_t n, int64_t k, const float *x,
                           const float *norm_w, float eps, uint16_t *h_out);
/* the attention-input chain of mi_qkv_rope_kv_q8_0 with Q4_0 weights (head_dim <= 128,
 * n[2] even) */
int mi_qkv_rope_kv_q4_0(void *stream, const void *const *w_packed, const int64_t *n, const float *const *bias,
                        int64_t k, const float *x, const float *norm_w, float eps, int64_t head_dim,
                        const int32_t *pos, float freq_base, float freq_scale, float attn_factor, float *q_out,
                        void *k_cache, size_t k_row_bytes, void *v_cache, size_t v_row_bytes, const void *kv_idx,
                        int kv_idx_is_i64, int64_t n_cache_rows, const float *rope_table);
/* the MUL_MAT of the ggml graph (src1 fp32): the activation is converted to fp16 (RNE, as
 * ggml converts src1) into LDS when m*k*2 <= 64 KB (no workspace), otherwise into ws of
 * mi_mul_mat_q4_0_workspace_size(m, k) bytes */
size_t mi_mul_mat_q4_0_workspace_size(int64_t m, int64_t k);
int mi_mul_mat_q4_0_f32(void *stream, const void *w_packed, const float *x, float *y, int64_t n, int64_t k,
                        int64_t m, void *ws, size_t ws_bytes);
/* fp32 -> fp16 round-to-nearest-even of n values (n % 4 == 0) */
int mi_cast_f32_f16(void *stream, const float *x, uint16_t *y, int64_t n);

/* The output head of a decode token with its graph neighbours folded in:
 * RMS_NORM(x) -> MUL(norm_w) -> MUL_MAT(F16 weight w [n rows of k, row stride ldw
 * elements]) -> ARGMAX.  Writes the logits y [n] (bit-identical to mi_rms_norm,
 * mi_gemv_f16 and mi_argmax in sequence) and their first maximum *out, in two launches:
 * the head with the norm in its prologue and ARGMAX's first pass in its epilogue, then
 * the final pass.  k a multiple of 32, at most 4096.  ws:
 * mi_head_f16_argmax_workspace_size(n, k) bytes.  Replaces the reference's separate
 * RMS_NORM, MUL and F16 MUL_MAT (patch:1133-1170, 1286-1309) and the host's greedy pick
 * over the logits. */
size_t mi_head_f16_argmax_workspace_size(int64_t n, int64_t k);
int mi_head_f16_argmax(void *stream, const uint16_t *w, int64_t ldw, const float *x, const float *norm_w, float eps,
                       float *y, int32_t *out, int64_t n, int64_t k, void *ws, size_t ws_bytes);
/* ------------------------------------------------------------------------
 * F16 GEMV (replaces cast + aclnnMatmul(FRACTAL_NZ) + cast, patch:1286-1309,
 * used for the tied output head).  w : fp16 rows, row stride ldw elements
 * (>= k, multiple of 8); x : fp32 [m][k], rounded to fp16 like ggml's
 * vec_dot_type conversion; y : fp32 [m][n]; fp32 accumulation (on the matrix cores
 * for m = 2..8 when k % 32 == 0 and m * (k + 8) * 2 <= 64 KiB).
 * ---------------------------------------------------------------------- */
int mi_gemv_f16(void *stream, const uint16_t *w, int64_t ldw, const float *x, float *y, int64_t n, int64_t k,
                int64_t m);

/* ------------------------------------------------------------------------
 * Single-token GQA flash-decoding (replaces AttentionStepCustom,
 * experiments/attention-step-custom/custom_ops/attention_step_custom.json:2-18,
 * op_host/attention_step_custom.cpp:80-121, and the q/out casts patch:1403,1426).
 * q    : fp32 [n_q_heads][d]
 * k, v : fp16, element (pos, kv_head, i) at byte offset pos*nb1 + kv_head*nb2 + 2*i
 *        (the ggml KV-cache view; strides multiples of 16 bytes)
 * mask : fp16 [n_kv] added to the scaled scores (-inf excludes), or NULL
 * kv_len: device int32[1], effective KV length (ggml src[5]); used when
 *        0 < *kv_len < n_kv, else n_kv; may be NULL
 * out  : fp32 [n_q_heads][d]
 * ws   : workspace of mi_fa_decode_workspace_size() bytes, 256-byte aligned (split partials and
 *        per-kv-head arrival counters); it must be zero-filled once before its first use and is
 *        left zeroed by every call, so calls sharing one workspace must be stream-ordered
 * d must be 64 or 128; n_q_heads % n_kv_heads == 0; group size <= 8 (<= 16 on the MFMA path).
 * ---------------------------------------------------------------------- */
size_t mi_fa_decode_workspace_size(int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d);
int mi_fa_decode(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                 const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                 size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out,
                 void *ws, size_t ws_bytes);
/* n_seq independent sequences in one launch (ggml FLASH_ATTN_EXT with one query row per
 * stream, ne[3] = n_seq: llama.cpp's per-sequence KV streams).  Sequence s uses
 * q + s*q_seq and out + s*out_seq (floats), k + s*k_seq and v + s*v_seq (bytes),
 * mask + s*mask_seq (elements) and kv_len[s].  No reference counterpart: the reference
 * decodes one sequence (patch:1957-1983 requires one query row). */
size_t mi_fa_decode_batch_workspace_size(int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                                         int64_t n_seq);
int mi_fa_decode_batch(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                       const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                       size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out,
                       int64_t n_seq, size_t q_seq, size_t k_seq, size_t v_seq, size_t mask_seq, size_t out_seq,
                       void *ws, size_t ws_bytes);
/* n_rows (1..8) query rows of ONE sequence in one launch: ggml FLASH_ATTN_EXT with
 * q ne[1] = n_rows (a prompt ubatch of llama.cpp, q permuted to [d, n_rows, n_q_heads]).
 * Every row reads the same K/V view and the same kv_len[0]; row r uses q + r*q_row and
 * out + r*out_row (floats, heads contiguous within a row) and mask + r*mask_row
 * (elements: llama.cpp's causal mask, one F16 row per query row).  Workspace:
 * mi_fa_decode_batch_workspace_size(..., n_rows).  No reference counterpart: the
 * reference's attention operator takes one query row (patch:1957-1983); this keeps a
 * one-sequence ubatch of up to 8 tokens on the device. */
int mi_fa_decode_rows(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                      const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                      size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out, int64_t n_rows,
                      size_t q_row, size_t mask_row, size_t out_row, void *ws, size_t ws_bytes);
/* mi_fa_decode_batch whose output goes straight to the input of the next several-row
 * W4A16 projection (mi_mul_mat_q4_0_batch_xp): sequence s's attention output row
 * (n_q_heads * d values, head-major) is written to xp as fp16 (RNE, ggml's src1
 * conversion) in that entry's permuted block layout; no fp32 output.  ws as for
 * mi_fa_decode_batch (required here even for one split).  No reference counterpart
 * (the reference decodes one sequence, patch:1957-1983). */
int mi_fa_decode_batch_q4act(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                             const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                             size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, void *xp,
                             int64_t n_seq, size_t q_seq, size_t k_seq, size_t v_seq, size_t mask_seq, void *ws,
                             size_t ws_bytes);
/* The split half of mi_fa_decode alone, for a consumer that merges the splits itself
 * (mi_mul_mat_q8_0_f32_lse): every split writes its record to ws and no combine runs.
 * Record of q head h, split s: floats ws[(h*S + s)*(d+4) + i], i < d: the unnormalised
 * output sum_j e^(s_j - m) v_j; [d]: m, the split's running maximum in log2 units
 * (scores times log2(e)), -inf for a split with no position; [d+1]: l = sum_j e^(s_j - m).
 * S = mi_fa_decode_num_splits(); ws as for mi_fa_decode (its size, 256-byte alignment).
 * No reference counterpart: the reference streams the whole KV length per head, no splits. */
int64_t mi_fa_decode_num_splits(int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d);
int mi_fa_decode_partials(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                          const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                          size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, void *ws,
                          size_t ws_bytes);
/* mi_fa_decode without a workspace argument, allocating nothing: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The split partials go
 * to a fixed per-device scratch array inside the library (mi_fa_decode_noalloc_max_workspace()
 * = 4 MiB, held until the process ends); a call whose mi_fa_decode_workspace_size exceeds
 * it fails with MI_ERR_WORKSPACE (12 q / 2 kv heads at D=128 fit up to ~400K positions,
 * 28 q / 4 kv up to 131K).  Every call on one device shares that array: calls that overlap
 * on one GPU (concurrent streams, or threads) race and must be serialised by the caller.
 * The stream must belong to the current device.  Results are bit-identical to mi_fa_decode. */
size_t mi_fa_decode_noalloc_max_workspace(void);
int mi_fa_decode_noalloc(void *stream, const float *q, const void *k, const void *v, const uint16_t *mask,
                         const int32_t *kv_len, int64_t n_kv, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                         size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale, float *out);

/* ------------------------------------------------------------------------
 * Decode-graph glue ops (one launch each; ggml-CPU semantics of
 * ggml/src/ggml-cpu/ops.cpp): the ops a llama.cpp decode graph places around
 * MUL_MAT and FLASH_ATTN_EXT, so that the whole token stays on the device.
 * ---------------------------------------------------------------------- */
/* y = x / sqrt(mean(x^2) + eps) [* w], rows of ne0 fp32 (ggml RMS_NORM [+ MUL]) */
int mi_rms_norm(void *stream, const float *x, const float *w, float *y, int64_t ne0, int64_t nrows, float eps);
/* d[i] = a[i] + b[i % nb] / a[i] * b[i % nb] (ggml ADD / MUL with row broadcast) */
int mi_add_bcast(void *stream, const float *a, const float *b, float *d, int64_t n, int64_t nb);
int mi_mul_bcast(void *stream, const float *a, const float *b, float *d, int64_t n, int64_t nb);
/* neox RoPE of x[ne2 tokens][ne1 heads][ne0] (byte strides nb1, nb2 in, ob1, ob2 out), pos[ne2] */
int mi_rope_neox(void *stream, const float *x, float *y, const int32_t *pos, int64_t ne0, int64_t ne1, int64_t ne2,
                 int64_t n_dims, float freq_base, float freq_scale, float attn_factor, size_t nb1, size_t nb2,
                 size_t ob1, size_t ob2);
/* ROPE q, ROPE k (neox over all head_dim dims; activation row r at position pos[r]), then
 * SET_ROWS of the rotated k and of v (fp32 -> fp16) into cache rows kv_idx[r] (skipped when
 * outside [0, n_cache_rows)): the four nodes after the q/k/v projections of a ubatch of m
 * tokens in one launch.  q [m][n_head_q*head_dim], k [m][n_head_k*head_dim], v [m][n_v]
 * fp32; q_out like q.  Per element the arithmetic of mi_rope_neox and mi_set_rows_f16.
 * Replaces the CANN RoPE and KV writes (patch:1360-1363, 1179-1184). */
int mi_rope_kv_rows(void *stream, const float *q, const float *k, const float *v, float *q_out, void *k_cache,
                    size_t k_row_bytes, void *v_cache, size_t v_row_bytes, const int32_t *pos, const void *kv_idx,
                    int kv_idx_is_i64, int64_t n_cache_rows, int64_t m, int64_t head_dim, int64_t n_head_q,
                    int64_t n_head_k, int64_t n_v, float freq_base, float freq_scale, float attn_factor);
/* the rotation table of mi_rope_neox for one position: table[p] = cos(theta_p) *
 * attn_factor, table[head_dim/2 + p] = sin(theta_p) * attn_factor (p < head_dim/2).  The
 * fused q/k/v chains take it instead of forming the angles per launch (the backend
 * builds it once per graph, as the CPU backend builds its rope cache once per node). */
int mi_rope_table(void *stream, const int32_t *pos, int64_t head_dim, float freq_base, float freq_scale,
                  float attn_factor, float *table);
/* fp16 table rows idx[r] = src row r (ggml SET_ROWS into the KV cache); idx int64 or int32 */
int mi_set_rows_f16(void *stream, const float *src, const void *idx, int idx_is_i64, uint16_t *dst, int64_t ne0,
                    int64_t nrows, size_t snb1, size_t dnb1, int64_t n_dst_rows);
/* dst row r = src row idx[r] as fp32 (ggml GET_ROWS, fp16 or fp32 table) */
int mi_get_rows(void *stream, const void *src, int src_is_f16, const int32_t *idx, float *dst, int64_t ne0,
                int64_t nrows, size_t snb1, int64_t n_src_rows);
/* d = silu(g) * u (ggml GLU SWIGLU, split form) */
int mi_swiglu(void *stream, const float *g, const float *u, float *d, int64_t n);
/* index of the first maximum of each row (ggml ARGMAX; the first maximum is what
 * llama.cpp's greedy sampler selects).  Two passes through a workspace of
 * mi_argmax_workspace_size bytes (8-byte aligned, no initial contents needed). */
size_t mi_argmax_workspace_size(int64_t ne0, int64_t nrows);
int mi_argmax(void *stream, const float *x, int32_t *out, int64_t ne0, int64_t nrows, void *ws, size_t ws_bytes);
/* decode mask row from a device length: 0 for i < *len, -inf beyond */
int mi_fill_mask_f16(void *stream, uint16_t *mask, const int32_t *len, int64_t n_kv);
/* rows x row_elems fp16 values uniform in [-scale, scale) (row stride in bytes), from a
 * counter-based hash of seed and the element index; synthetic KV-cache contents */
int mi_fill_f16_uniform(void *stream, void *dst, int64_t rows, int64_t row_elems, size_t row_stride, uint64_t seed,
                        float scale);

/* ------------------------------------------------------------------------
 * kv_lengths on the device (replaces the host scan set_input_kv_lengths,
 * patch:2900-2929): out[r] = max(1, 1 + last index with a finite mask value).
 * ---------------------------------------------------------------------- */
int mi_kv_lengths(void *stream, const void *mask, int mask_is_f16, int64_t n_kv, int64_t n_rows, int32_t *out);

#ifdef __cplusplus
}
#endif
#endif

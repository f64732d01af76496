// qwen2.cpp -- minimal Qwen2 decode driver over the ggml backend API (see mi_qwen2.h).
//
// Graph per step, following llama.cpp's Qwen2 builder: GET_ROWS(token_embd) ->
// n_layer x [RMS_NORM, MUL, q/k/v MUL_MAT (+bias ADD), ROPE neox, SET_ROWS K/V into the
// fp16 cache, FLASH_ATTN_EXT (+kv_lengths src[5]), MUL_MAT o, ADD residual,
// RMS_NORM, MUL, gate/up MUL_MAT, GLU swiglu, MUL_MAT down, ADD residual] ->
// RMS_NORM, MUL, MUL_MAT(tied token_embd) -> ARGMAX.  A step decodes one token for
// each of n_seq independent sequences (one ubatch of n_seq tokens).  Each sequence
// owns n_ctx rows of every layer's cache; the attention sees the caches as n_seq
// streams (ggml ne[3]), as llama.cpp's per-sequence KV streams.  The KV view covers
// the longest used cache rounded up to 256 positions (as llama.cpp's KV view is), so
// one graph serves 256 consecutive positions and the backend replays it as a captured
// HIP graph.
#include "mi_qwen2.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include <hip/hip_runtime.h>

#include "ggml-backend.h"
#include "ggml-mi355x.h"
#include "ggml.h"
#include "ggml_mi355x_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

constexpr int kMaxUbatch = 8;                      // prompt tokens per ubatch (the MUL_MAT row limit)
constexpr int kPromptWords = 3 * kMaxUbatch + 2;  // pinned prompt inputs + the greedy token read back

struct Graph {
    int n_kv = 0;  // KV view length
    ggml_context *ctx = nullptr;
    ggml_cgraph *gf = nullptr;
    ggml_gallocr_t galloc = nullptr;
    ggml_tensor *logits = nullptr;
    ggml_tensor *argmax = nullptr;
    std::vector<ggml_tensor *> l_out;  // each layer's output (the residual stream), F32 [n_embd, n_seq]
    // with the layer dump on: each layer's normed FFN input and FFN output, F32 [n_embd, n_seq]
    std::vector<ggml_tensor *> ffn_norm, ffn_out;
};

}  // namespace

struct mi_qwen2 {
    mi_qwen2_hparams hp;
    int n_seq = 1;
    ggml_backend_t backend = nullptr;
    ggml_context *wctx = nullptr;
    ggml_backend_buffer_t wbuf = nullptr;
    std::map<std::string, ggml_tensor *> tensors;
    std::vector<ggml_tensor *> k_cache, v_cache;  // F16 [n_embd_kv, n_ctx * n_seq]
    ggml_tensor *inp = nullptr;  // I32 [4 * n_seq]: tokens, positions, kv lengths, cache rows
    // pinned host words: the 4 * n_seq inputs, then the n_seq greedy tokens read back
    // (asynchronous copies on the backend's stream)
    int32_t *io_pinned = nullptr;
    // MI_QWEN2_KQ_MASK=1 (one sequence): the attention also takes llama.cpp's KQ mask, F16
    // [n_ctx] (0 up to the token's position, -inf after it), beside the kv lengths, as the
    // reference's patched llama.cpp graph passes both.  MI_QWEN2_KQ_MASK=swa:N keeps only
    // the last N positions (a sliding-window mask, as llama.cpp builds for SWA layers).
    bool use_mask = false;
    int32_t mask_window = 0;  // 0: causal only
    ggml_tensor *mask = nullptr;
    uint16_t *mask_pinned = nullptr;
    // prompt ubatches (mi_qwen2_prefill): I32 [3 * 8 + 1] tokens, positions, the kv length,
    // cache rows; the causal mask F16 [n_kv, T] of the ubatch (up to n_ctx x 8)
    ggml_tensor *inp_pf = nullptr, *mask_pf = nullptr;
    uint16_t *mask_pf_pinned = nullptr;
    std::map<int, Graph> graphs;  // by KV view length
    std::map<std::tuple<int, int, int>, Graph> pgraphs;  // prompt ubatches: (KV view, rows, sequence)
    Graph *last = nullptr;        // the graph of the latest decode step
    bool dump = false;            // graphs keep ffn_norm-N / ffn_out-N as outputs
};

namespace {

ggml_tensor *W(mi_qwen2 *m, const std::string &name) {
    auto it = m->tensors.find(name);
    if (it == m->tensors.end()) GGML_ABORT("qwen2: missing tensor %s", name.c_str());
    return it->second;
}

ggml_tensor *add_tensor(mi_qwen2 *m, const std::string &name, ggml_type type, int64_t ne0, int64_t ne1 = 1) {
    ggml_tensor *t = ne1 == 1 ? ggml_new_tensor_1d(m->wctx, type, ne0) : ggml_new_tensor_2d(m->wctx, type, ne0, ne1);
    ggml_set_name(t, name.c_str());
    m->tensors[name] = t;
    return t;
}

// One decode step of every sequence (T = 0: S = n_seq streams of one token each), or a
// prompt ubatch of T tokens of sequence `seq` (one stream; FLASH_ATTN_EXT with T query
// rows and llama.cpp's causal mask, one mask row per token; logits of the last token).
Graph build_graph(mi_qwen2 *m, int n_kv, int T = 0, int seq = 0) {
    const mi_qwen2_hparams &hp = m->hp;
    const bool prompt = T > 0;
    const int S = prompt ? 1 : m->n_seq;  // KV streams
    if (!prompt) T = 1;
    const int R = S * T;                  // activation rows
    const int hd = hp.head_dim, n_embd_kv = hp.n_head_kv * hd;
    Graph G;
    G.n_kv = n_kv;
    ggml_init_params ip = {0, nullptr, true};
    G.ctx = ggml_init(ip);
    ggml_context *ctx = G.ctx;
    ggml_cgraph *gf = ggml_new_graph_custom(ctx, 16384, false);
    G.gf = gf;

    // inputs: R tokens, R positions, S kv lengths, R cache rows
    ggml_tensor *in = prompt ? m->inp_pf : m->inp;
    ggml_tensor *tok = ggml_view_1d(ctx, in, R, 0);
    ggml_tensor *pos = ggml_view_1d(ctx, in, R, 4 * (size_t)R);
    ggml_tensor *kvl = ggml_view_1d(ctx, in, S, 8 * (size_t)R);
    ggml_tensor *kidx = ggml_view_1d(ctx, in, R, 8 * (size_t)R + 4 * (size_t)S);
    ggml_tensor *tok_embd = W(m, "token_embd.weight");

    ggml_tensor *inpL = ggml_get_rows(ctx, tok_embd, tok);
    const float kq_scale = 1.0f / sqrtf((float)hd);
    for (int il = 0; il < hp.n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        ggml_tensor *cur = ggml_rms_norm(ctx, inpL, hp.rms_eps);
        cur = ggml_mul(ctx, cur, W(m, p + "attn_norm.weight"));
        ggml_tensor *Q = ggml_mul_mat(ctx, W(m, p + "attn_q.weight"), cur);
        ggml_tensor *K = ggml_mul_mat(ctx, W(m, p + "attn_k.weight"), cur);
        ggml_tensor *V = ggml_mul_mat(ctx, W(m, p + "attn_v.weight"), cur);
        ggml_build_forward_expand(gf, Q);  // q/k/v projections adjacent in node order
        ggml_build_forward_expand(gf, K);
        ggml_build_forward_expand(gf, V);
        if (hp.use_bias) {
            Q = ggml_add(ctx, Q, W(m, p + "attn_q.bias"));
            K = ggml_add(ctx, K, W(m, p + "attn_k.bias"));
            V = ggml_add(ctx, V, W(m, p + "attn_v.bias"));
            ggml_build_forward_expand(gf, Q);  // bias adds adjacent, in q/k/v order
            ggml_build_forward_expand(gf, K);
            ggml_build_forward_expand(gf, V);
        }
        Q = ggml_reshape_3d(ctx, Q, hd, hp.n_head, R);
        K = ggml_reshape_3d(ctx, K, hd, hp.n_head_kv, R);
        Q = ggml_rope_ext(ctx, Q, pos, nullptr, hd, GGML_ROPE_TYPE_NEOX, 0, hp.rope_theta, 1.0f, 0.0f, 1.0f, 0.0f,
                          0.0f);
        K = ggml_rope_ext(ctx, K, pos, nullptr, hd, GGML_ROPE_TYPE_NEOX, 0, hp.rope_theta, 1.0f, 0.0f, 1.0f, 0.0f,
                          0.0f);
        ggml_build_forward_expand(gf, Q);  // rope q, rope k, then the two cache writes: the
        ggml_build_forward_expand(gf, K);  // attention-input chain the backend fuses
        ggml_tensor *kc = m->k_cache[il], *vc = m->v_cache[il];
        ggml_build_forward_expand(gf, ggml_set_rows(ctx, kc, ggml_reshape_2d(ctx, K, n_embd_kv, R), kidx));
        ggml_build_forward_expand(gf, ggml_set_rows(ctx, vc, V, kidx));
        // sequence s's cache is rows [s*n_ctx, (s+1)*n_ctx): stream s of the 4-D view
        const size_t seq_bytes = (size_t)hp.n_ctx * kc->nb[1];
        const size_t seq_off = prompt ? (size_t)seq * seq_bytes : 0;
        ggml_tensor *k = ggml_view_4d(ctx, kc, hd, n_kv, hp.n_head_kv, S, kc->nb[1], ggml_row_size(GGML_TYPE_F16, hd),
                                      seq_bytes, seq_off);
        ggml_tensor *v = ggml_view_4d(ctx, vc, hd, n_kv, hp.n_head_kv, S, vc->nb[1], ggml_row_size(GGML_TYPE_F16, hd),
                                      seq_bytes, seq_off);
        // q [hd, T, n_head, S], as llama.cpp permutes it for FLASH_ATTN_EXT
        ggml_tensor *q = ggml_permute(ctx, ggml_reshape_4d(ctx, Q, hd, hp.n_head, T, S), 0, 2, 1, 3);
        ggml_tensor *kq_mask = prompt   ? ggml_view_2d(ctx, m->mask_pf, n_kv, T, (size_t)n_kv * 2, 0)
                               : m->mask ? ggml_view_1d(ctx, m->mask, n_kv, 0)
                                         : nullptr;
        ggml_tensor *att = ggml_flash_attn_ext(ctx, q, k, v, kq_mask, kq_scale, 0.0f, 0.0f);
        ggml_flash_attn_ext_add_kv_lengths(att, kvl);
        ggml_flash_attn_ext_set_prec(att, GGML_PREC_F32);
        cur = ggml_reshape_2d(ctx, att, hd * hp.n_head, R);
        cur = ggml_mul_mat(ctx, W(m, p + "attn_output.weight"), cur);
        ggml_tensor *ffn_inp = ggml_add(ctx, cur, inpL);
        cur = ggml_rms_norm(ctx, ffn_inp, hp.rms_eps);
        cur = ggml_mul(ctx, cur, W(m, p + "ffn_norm.weight"));
        if (m->dump) {  // named as llama.cpp's graph callback names them; outputs, so no fusion skips them
            ggml_set_name(cur, ("ffn_norm-" + std::to_string(il)).c_str());
            ggml_set_output(cur);
            G.ffn_norm.push_back(cur);
        }
        ggml_tensor *g = ggml_mul_mat(ctx, W(m, p + "ffn_gate.weight"), cur);
        ggml_tensor *u = ggml_mul_mat(ctx, W(m, p + "ffn_up.weight"), cur);
        ggml_build_forward_expand(gf, g);  // gate/up adjacent
        ggml_build_forward_expand(gf, u);
        cur = ggml_swiglu_split(ctx, g, u);
        cur = ggml_mul_mat(ctx, W(m, p + "ffn_down.weight"), cur);
        if (m->dump) {
            ggml_set_name(cur, ("ffn_out-" + std::to_string(il)).c_str());
            ggml_set_output(cur);
            G.ffn_out.push_back(cur);
        }
        inpL = ggml_add(ctx, cur, ffn_inp);
        ggml_set_name(inpL, ("l_out-" + std::to_string(il)).c_str());  // the eval-callback name
        G.l_out.push_back(inpL);
    }
    // a prompt ubatch's logits: its last token only (llama.cpp's output ids)
    if (prompt && T > 1) inpL = ggml_view_2d(ctx, inpL, hp.n_embd, 1, inpL->nb[1], (size_t)(T - 1) * inpL->nb[1]);
    ggml_tensor *cur = ggml_rms_norm(ctx, inpL, hp.rms_eps);
    cur = ggml_mul(ctx, cur, W(m, "output_norm.weight"));
    G.logits = ggml_mul_mat(ctx, tok_embd, cur);  // tied output head
    G.argmax = ggml_argmax(ctx, G.logits);
    ggml_build_forward_expand(gf, G.argmax);

    G.galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(m->backend));
    if (!ggml_gallocr_alloc_graph(G.galloc, gf)) GGML_ABORT("qwen2: graph allocation failed");
    // every node must run on the backend (there is no CPU fallback in this driver)
    for (int i = 0; i < ggml_graph_n_nodes(gf); i++) {
        ggml_tensor *n = ggml_graph_node(gf, i);
        if (!ggml_backend_supports_op(m->backend, n))
            GGML_ABORT("qwen2: backend does not support node %s (%s)", n->name, ggml_op_name(n->op));
    }
    return G;
}

Graph &graph_for(mi_qwen2 *m, int32_t kv_len) {
    int n_kv = (kv_len + 255) / 256 * 256;
    if (n_kv > m->hp.n_ctx) n_kv = m->hp.n_ctx;
    auto it = m->graphs.find(n_kv);
    if (it != m->graphs.end()) return it->second;
    return m->graphs.emplace(n_kv, build_graph(m, n_kv)).first->second;
}

Graph &prompt_graph_for(mi_qwen2 *m, int32_t kv_len, int T, int seq) {
    int n_kv = (kv_len + 255) / 256 * 256;
    if (n_kv > m->hp.n_ctx) n_kv = m->hp.n_ctx;
    const auto key = std::make_tuple(n_kv, T, seq);
    auto it = m->pgraphs.find(key);
    if (it != m->pgraphs.end()) return it->second;
    return m->pgraphs.emplace(key, build_graph(m, n_kv, T, seq)).first->second;
}

int check_cache_args(mi_qwen2 *m, int32_t layer, int32_t seq, int32_t n_pos) {
    if (layer < 0 || layer >= m->hp.n_layer) return fail("qwen2: layer %d out of range", layer);
    if (seq < 0 || seq >= m->n_seq) return fail("qwen2: sequence %d out of range", seq);
    if (n_pos < 0 || n_pos > m->hp.n_ctx) return fail("qwen2: n_pos %d outside the cache", n_pos);
    return 0;
}

}  // namespace

extern "C" {

const char *mi_qwen2_last_error(void) { return g_err; }

mi_qwen2 *mi_qwen2_create(const mi_qwen2_hparams *hp, int device) {
    if (!hp || hp->n_layer <= 0 || hp->n_embd <= 0 || hp->n_head <= 0 || hp->n_head_kv <= 0 ||
        hp->n_head % hp->n_head_kv != 0 || hp->head_dim * hp->n_head != hp->n_embd || hp->n_ctx <= 0 ||
        hp->n_seq < 0 || hp->n_seq > 8 ||
        (hp->wtype != GGML_TYPE_Q8_0 && hp->wtype != GGML_TYPE_Q4_0 && hp->wtype != GGML_TYPE_F16)) {
        fail("qwen2: invalid hyper-parameters");
        return nullptr;
    }
    mi_qwen2 *m = new mi_qwen2();
    m->hp = *hp;
    m->n_seq = hp->n_seq > 0 ? hp->n_seq : 1;
    m->hp.n_seq = m->n_seq;
    m->backend = ggml_backend_mi355x_init(device);
    if (!m->backend) {
        delete m;
        fail("qwen2: no MI355X device %d", device);
        return nullptr;
    }
    if (hipHostMalloc((void **)&m->io_pinned, (5 * (size_t)m->n_seq + kPromptWords) * sizeof(int32_t),
                      hipHostMallocDefault) !=
        hipSuccess) {
        ggml_backend_free(m->backend);
        delete m;
        fail("qwen2: pinned host allocation failed");
        return nullptr;
    }
    ggml_init_params ip = {0, nullptr, true};
    m->wctx = ggml_init(ip);
    const ggml_type wt = (ggml_type)hp->wtype;
    const int n_embd_kv = hp->n_head_kv * hp->head_dim;
    add_tensor(m, "token_embd.weight", GGML_TYPE_F16, hp->n_embd, hp->n_vocab);
    add_tensor(m, "output_norm.weight", GGML_TYPE_F32, hp->n_embd);
    for (int il = 0; il < hp->n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        add_tensor(m, p + "attn_norm.weight", GGML_TYPE_F32, hp->n_embd);
        add_tensor(m, p + "attn_q.weight", wt, hp->n_embd, hp->n_embd);
        add_tensor(m, p + "attn_k.weight", wt, hp->n_embd, n_embd_kv);
        add_tensor(m, p + "attn_v.weight", wt, hp->n_embd, n_embd_kv);
        if (hp->use_bias) {
            add_tensor(m, p + "attn_q.bias", GGML_TYPE_F32, hp->n_embd);
            add_tensor(m, p + "attn_k.bias", GGML_TYPE_F32, n_embd_kv);
            add_tensor(m, p + "attn_v.bias", GGML_TYPE_F32, n_embd_kv);
        }
        add_tensor(m, p + "attn_output.weight", wt, hp->n_embd, hp->n_embd);
        add_tensor(m, p + "ffn_norm.weight", GGML_TYPE_F32, hp->n_embd);
        add_tensor(m, p + "ffn_gate.weight", wt, hp->n_embd, hp->n_ff);
        add_tensor(m, p + "ffn_up.weight", wt, hp->n_embd, hp->n_ff);
        add_tensor(m, p + "ffn_down.weight", wt, hp->n_ff, hp->n_embd);
        ggml_tensor *kc = ggml_new_tensor_2d(m->wctx, GGML_TYPE_F16, n_embd_kv, (int64_t)hp->n_ctx * m->n_seq);
        ggml_tensor *vc = ggml_new_tensor_2d(m->wctx, GGML_TYPE_F16, n_embd_kv, (int64_t)hp->n_ctx * m->n_seq);
        ggml_set_name(kc, ("cache_k_l" + std::to_string(il)).c_str());
        ggml_set_name(vc, ("cache_v_l" + std::to_string(il)).c_str());
        m->k_cache.push_back(kc);
        m->v_cache.push_back(vc);
    }
    m->inp = ggml_new_tensor_1d(m->wctx, GGML_TYPE_I32, 4 * (int64_t)m->n_seq);
    ggml_set_name(m->inp, "inp_decode");
    ggml_set_input(m->inp);
    m->inp_pf = ggml_new_tensor_1d(m->wctx, GGML_TYPE_I32, 3 * kMaxUbatch + 1);
    ggml_set_name(m->inp_pf, "inp_prompt");
    ggml_set_input(m->inp_pf);
    m->mask_pf = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F16, (int64_t)hp->n_ctx * kMaxUbatch);
    ggml_set_name(m->mask_pf, "inp_kq_mask_prompt");
    ggml_set_input(m->mask_pf);
    {
        const char *e = getenv("MI_QWEN2_KQ_MASK");
        if (e && !strncmp(e, "swa:", 4)) m->mask_window = std::max(1, atoi(e + 4));
        m->use_mask = e && (e[0] == '1' || m->mask_window > 0) && m->n_seq == 1;
    }
    if (m->use_mask) {
        m->mask = ggml_new_tensor_1d(m->wctx, GGML_TYPE_F16, hp->n_ctx);
        ggml_set_name(m->mask, "inp_kq_mask");
        ggml_set_input(m->mask);
    }
    m->wbuf = ggml_backend_alloc_ctx_tensors_from_buft(m->wctx, ggml_backend_mi355x_buffer_type(device));
    if (!m->wbuf) {
        mi_qwen2_free(m);
        fail("qwen2: weight buffer allocation failed");
        return nullptr;
    }
    ggml_backend_buffer_set_usage(m->wbuf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    if ((m->mask && hipHostMalloc((void **)&m->mask_pinned, (size_t)hp->n_ctx * 2, hipHostMallocDefault) != hipSuccess) ||
        hipHostMalloc((void **)&m->mask_pf_pinned, (size_t)hp->n_ctx * kMaxUbatch * 2, hipHostMallocDefault) !=
            hipSuccess) {
        mi_qwen2_free(m);
        fail("qwen2: pinned host allocation failed");
        return nullptr;
    }
    mi_qwen2_reset(m);
    return m;
}

void mi_qwen2_free(mi_qwen2 *m) {
    if (!m) return;
    for (auto &kv : m->graphs) {
        ggml_gallocr_free(kv.second.galloc);
        ggml_free(kv.second.ctx);
    }
    for (auto &kv : m->pgraphs) {
        ggml_gallocr_free(kv.second.galloc);
        ggml_free(kv.second.ctx);
    }
    ggml_backend_buffer_free(m->wbuf);
    ggml_free(m->wctx);
    ggml_backend_free(m->backend);
    if (m->io_pinned) (void)hipHostFree(m->io_pinned);
    if (m->mask_pinned) (void)hipHostFree(m->mask_pinned);
    if (m->mask_pf_pinned) (void)hipHostFree(m->mask_pf_pinned);
    delete m;
}

int mi_qwen2_reset(mi_qwen2 *m) {
    for (size_t i = 0; i < m->k_cache.size(); i++) {
        ggml_backend_tensor_memset(m->k_cache[i], 0, 0, ggml_nbytes(m->k_cache[i]));
        ggml_backend_tensor_memset(m->v_cache[i], 0, 0, ggml_nbytes(m->v_cache[i]));
    }
    return 0;
}

int32_t mi_qwen2_n_seq(const mi_qwen2 *m) { return m->n_seq; }

int64_t mi_qwen2_tensor_nbytes(mi_qwen2 *m, const char *name, int64_t *dims) {
    auto it = m->tensors.find(name);
    if (it == m->tensors.end()) return -1;
    if (dims) {
        dims[0] = it->second->ne[0];
        dims[1] = it->second->ne[1];
    }
    return (int64_t)ggml_nbytes(it->second);
}

int mi_qwen2_set_tensor(mi_qwen2 *m, const char *name, const void *data, size_t size) {
    auto it = m->tensors.find(name);
    if (it == m->tensors.end()) return fail("qwen2: unknown tensor %s", name);
    if (size != ggml_nbytes(it->second))
        return fail("qwen2: %s expects %zu bytes, got %zu", name, ggml_nbytes(it->second), size);
    ggml_backend_tensor_set(it->second, data, 0, size);
    return 0;
}

int mi_qwen2_set_smooth(mi_qwen2 *m, const char *weight_name, const float *s, int64_t n) {
    auto it = m->tensors.find(weight_name);
    if (it == m->tensors.end()) return fail("qwen2: unknown tensor %s", weight_name);
    if (!ggml_backend_mi355x_set_smooth_factors(it->second, s, n))
        return fail("qwen2: %s takes no SmoothQuant factors of length %lld", weight_name, (long long)n);
    return 0;
}

int mi_smooth_scales_read(const char *path, int64_t n_layer, int64_t n_embd, float *out) {
    if (!path || !out || n_layer <= 0 || n_embd <= 0) return fail("smooth scales: bad arguments");
    FILE *f = fopen(path, "rb");
    if (!f) return fail("smooth scales: cannot open %s", path);
    const size_t want = (size_t)n_layer * (size_t)n_embd;
    long size = -1;
    if (fseek(f, 0, SEEK_END) == 0) size = ftell(f);
    if (size != (long)(want * sizeof(float))) {
        fclose(f);
        return fail("smooth scales: %s holds %ld bytes, expected %zu (fp32 [%lld layers][%lld])", path, size,
                    want * sizeof(float), (long long)n_layer, (long long)n_embd);
    }
    rewind(f);
    const size_t got = fread(out, sizeof(float), want, f);  // little-endian fp32, as the file is written
    fclose(f);
    if (got != want) return fail("smooth scales: short read of %s", path);
    for (size_t i = 0; i < want; i++)
        if (!(out[i] > 0.0f) || !isfinite(out[i]))
            return fail("smooth scales: entry %zu (layer %zu, channel %zu) is %g, not a positive finite factor", i,
                        i / (size_t)n_embd, i % (size_t)n_embd, (double)out[i]);
    return 0;
}

int mi_qwen2_load_smooth_file(mi_qwen2 *m, const char *path, int weights_presmoothed) {
    const int64_t L = m->hp.n_layer, E = m->hp.n_embd;
    if (m->hp.wtype == GGML_TYPE_Q8_0 && !weights_presmoothed)
        return fail("smooth scales: the Q8_0 FFN weights must already hold W*diag(s) (quantized from the smoothed "
                    "weights); pass weights_presmoothed = 1 to assert that, or load F16 weights with "
                    "GGML_MI355X_A8W8=1 so the backend folds s in at upload");
    std::vector<float> s((size_t)(L * E));
    if (int r = mi_smooth_scales_read(path, L, E, s.data())) return r;
    for (int64_t il = 0; il < L; il++)
        for (const char *w : {"ffn_gate", "ffn_up"}) {
            const std::string name = "blk." + std::to_string(il) + "." + w + ".weight";
            if (int r = mi_qwen2_set_smooth(m, name.c_str(), s.data() + il * E, E)) return r;
        }
    return 0;
}

int mi_qwen2_set_layer_dump(mi_qwen2 *m, int on) {
    if (m->dump == (on != 0)) return 0;
    m->dump = on != 0;
    for (auto &kv : m->graphs) {  // rebuilt on demand with the new outputs
        ggml_gallocr_free(kv.second.galloc);
        ggml_free(kv.second.ctx);
    }
    m->graphs.clear();
    m->last = nullptr;
    return 0;
}

int mi_qwen2_dump_layers(mi_qwen2 *m, const char *path, int append) {
    if (!path) return fail("qwen2: layer dump path is NULL");
    if (!m->last) return fail("qwen2: no decode step to dump");
    FILE *f = fopen(path, append ? "ab" : "wb");
    if (!f) return fail("qwen2: cannot open layer dump %s", path);
    bool ok = fseek(f, 0, SEEK_END) == 0;
    const long at = ok ? ftell(f) : -1;
    static const char magic[8] = {'L', 'L', 'D', 'U', 'M', 'P', '1', '\0'};
    if (at == 0) ok = fwrite(magic, 1, 8, f) == 8;
    else ok = ok && at >= 8;  // appending to a file that must already hold the header
    std::vector<ggml_tensor *> recs;  // graph order: per layer ffn_norm, ffn_out (dump mode), l_out
    for (size_t i = 0; i < m->last->l_out.size(); i++) {
        if (i < m->last->ffn_norm.size()) recs.push_back(m->last->ffn_norm[i]);
        if (i < m->last->ffn_out.size()) recs.push_back(m->last->ffn_out[i]);
        recs.push_back(m->last->l_out[i]);
    }
    std::vector<float> v;
    for (size_t i = 0; ok && i < recs.size(); i++) {
        ggml_tensor *t = recs[i];
        const uint64_t n = (uint64_t)ggml_nelements(t);
        const uint16_t nl = (uint16_t)strlen(t->name);
        v.resize(n);
        ggml_backend_tensor_get(t, v.data(), 0, n * sizeof(float));
        ok = fwrite(&nl, sizeof nl, 1, f) == 1 && fwrite(t->name, 1, nl, f) == nl && fwrite(&n, sizeof n, 1, f) == 1 &&
             fwrite(v.data(), sizeof(float), n, f) == n;
    }
    ok = (fclose(f) == 0) && ok;
    return ok ? 0 : fail("qwen2: writing layer dump %s failed", path);
}

int mi_qwen2_decode_batch(mi_qwen2 *m, const int32_t *tokens, const int32_t *pos, int32_t *next_tokens,
                          float *logits) {
    const int S = m->n_seq;
    if (!tokens || !pos) return fail("qwen2: tokens/positions are NULL");
    int32_t max_len = 0;
    for (int s = 0; s < S; s++) {
        if (pos[s] < 0 || pos[s] >= m->hp.n_ctx)
            return fail("qwen2: position %d of sequence %d outside the cache (%d)", pos[s], s, m->hp.n_ctx);
        if (tokens[s] < 0 || tokens[s] >= m->hp.n_vocab)
            return fail("qwen2: token %d of sequence %d outside the vocabulary", tokens[s], s);
        max_len = std::max(max_len, pos[s] + 1);
    }
    Graph &G = graph_for(m, max_len);
    int32_t *in = m->io_pinned, *out = m->io_pinned + 4 * S;
    for (int s = 0; s < S; s++) {
        in[s] = tokens[s];
        in[S + s] = pos[s];
        in[2 * S + s] = pos[s] + 1;
        in[3 * S + s] = s * m->hp.n_ctx + pos[s];
    }
    // inputs in, graph, greedy tokens out: one stream, one synchronisation
    ggml_backend_tensor_set_async(m->backend, m->inp, in, 0, 4 * (size_t)S * sizeof(int32_t));
    if (m->mask) {  // fp16 0 over the kept positions, -inf elsewhere
        const int32_t lo = m->mask_window > 0 ? pos[0] - m->mask_window + 1 : 0;
        for (int32_t j = 0; j < m->hp.n_ctx; j++) m->mask_pinned[j] = j <= pos[0] && j >= lo ? 0x0000 : 0xFC00;
        ggml_backend_tensor_set_async(m->backend, m->mask, m->mask_pinned, 0, (size_t)m->hp.n_ctx * 2);
    }
    if (ggml_backend_graph_compute(m->backend, G.gf) != GGML_STATUS_SUCCESS) return fail("qwen2: graph failed");
    if (next_tokens) ggml_backend_tensor_get_async(m->backend, G.argmax, out, 0, (size_t)S * sizeof(int32_t));
    if (ggml_backend_mi355x_status(m->backend) != 0) return fail("qwen2: decode failed: %s", mi_last_error());
    m->last = &G;
    if (next_tokens) memcpy(next_tokens, out, (size_t)S * sizeof(int32_t));
    if (logits) ggml_backend_tensor_get(G.logits, logits, 0, ggml_nbytes(G.logits));
    return 0;
}

int mi_qwen2_decode(mi_qwen2 *m, int32_t token, int32_t pos, int32_t *next_token, float *logits) {
    if (m->n_seq != 1) return fail("qwen2: mi_qwen2_decode needs n_seq == 1 (use mi_qwen2_decode_batch)");
    return mi_qwen2_decode_batch(m, &token, &pos, next_token, logits);
}

int mi_qwen2_decode_steps_batch(mi_qwen2 *m, const int32_t *tokens, const int32_t *pos, int32_t n_steps,
                                int32_t *out_tokens, double *seconds) {
    const int S = m->n_seq;
    if (n_steps < 0 || !tokens || !pos) return fail("qwen2: bad decode range");
    for (int s = 0; s < S; s++)
        if (pos[s] < 0 || pos[s] + n_steps > m->hp.n_ctx) return fail("qwen2: bad decode range");
    if (n_steps > 0 && !out_tokens) return fail("qwen2: out_tokens is NULL");
    std::vector<int32_t> cur(tokens, tokens + S), p(pos, pos + S), nxt(S);
    const auto t0 = std::chrono::steady_clock::now();
    for (int32_t i = 0; i < n_steps; i++) {
        if (mi_qwen2_decode_batch(m, cur.data(), p.data(), nxt.data(), nullptr)) return -1;
        for (int s = 0; s < S; s++) {
            out_tokens[(size_t)i * S + s] = nxt[s];
            cur[s] = nxt[s];
            p[s]++;
        }
    }
    const auto t1 = std::chrono::steady_clock::now();
    if (seconds) *seconds = std::chrono::duration<double>(t1 - t0).count();
    return 0;
}

int mi_qwen2_decode_steps(mi_qwen2 *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out_tokens,
                          double *seconds) {
    if (m->n_seq != 1) return fail("qwen2: mi_qwen2_decode_steps needs n_seq == 1");
    return mi_qwen2_decode_steps_batch(m, &token, &pos, n_steps, out_tokens, seconds);
}

int mi_qwen2_prefill(mi_qwen2 *m, int32_t seq, const int32_t *tokens, int32_t n_tokens, int32_t pos0,
                     int32_t n_ubatch, int32_t *next_token, float *logits, double *seconds) {
    if (!m || !tokens) return fail("qwen2: prefill: null argument");
    if (seq < 0 || seq >= m->n_seq) return fail("qwen2: prefill: sequence %d of %d", seq, m->n_seq);
    if (n_ubatch < 1 || n_ubatch > kMaxUbatch) return fail("qwen2: prefill: ubatch of %d tokens (1..%d)", n_ubatch,
                                                           kMaxUbatch);
    if (n_tokens < 1 || pos0 < 0 || pos0 + n_tokens > m->hp.n_ctx)
        return fail("qwen2: prefill: positions %d..%d outside the cache (%d)", pos0, pos0 + n_tokens - 1, m->hp.n_ctx);
    for (int32_t i = 0; i < n_tokens; i++)
        if (tokens[i] < 0 || tokens[i] >= m->hp.n_vocab) return fail("qwen2: prefill: token %d outside the vocabulary",
                                                                     tokens[i]);
    int32_t *in = m->io_pinned + 5 * (size_t)m->n_seq, *out = in + 3 * kMaxUbatch + 1;
    const auto t0 = std::chrono::steady_clock::now();
    Graph *G = nullptr;
    for (int32_t done = 0; done < n_tokens;) {
        const int T = std::min(n_ubatch, n_tokens - done);
        const int32_t p0 = pos0 + done, kv_len = p0 + T;
        G = &prompt_graph_for(m, kv_len, T, seq);
        const int64_t n_kv = G->n_kv;
        for (int t = 0; t < T; t++) {
            in[t] = tokens[done + t];
            in[T + t] = p0 + t;
            in[2 * T + 1 + t] = seq * m->hp.n_ctx + p0 + t;
        }
        in[2 * T] = kv_len;
        // causal: token t sees positions <= p0 + t (fp16 0), not the later ones (-inf)
        for (int t = 0; t < T; t++)
            for (int64_t j = 0; j < n_kv; j++) m->mask_pf_pinned[t * n_kv + j] = j <= p0 + t ? 0x0000 : 0xFC00;
        ggml_backend_tensor_set_async(m->backend, m->inp_pf, in, 0, (3 * (size_t)T + 1) * sizeof(int32_t));
        ggml_backend_tensor_set_async(m->backend, m->mask_pf, m->mask_pf_pinned, 0, (size_t)T * n_kv * 2);
        if (ggml_backend_graph_compute(m->backend, G->gf) != GGML_STATUS_SUCCESS) return fail("qwen2: graph failed");
        done += T;
        if (done == n_tokens && next_token)
            ggml_backend_tensor_get_async(m->backend, G->argmax, out, 0, sizeof(int32_t));
        // one synchronisation per ubatch: the pinned inputs are rewritten for the next one
        if (ggml_backend_mi355x_status(m->backend) != 0) return fail("qwen2: prefill failed: %s", mi_last_error());
    }
    const auto t1 = std::chrono::steady_clock::now();
    if (seconds) *seconds = std::chrono::duration<double>(t1 - t0).count();
    m->last = G;
    if (next_token) *next_token = out[0];
    if (logits) ggml_backend_tensor_get(G->logits, logits, 0, ggml_nbytes(G->logits));
    return 0;
}

int mi_qwen2_generate(mi_qwen2 *m, const int32_t *prompt, int32_t n_prompt, int32_t n_gen, int32_t *out_tokens,
                      double *gen_seconds) {
    if (m->n_seq != 1) return fail("qwen2: mi_qwen2_generate needs n_seq == 1");
    if (!prompt || n_prompt < 1 || n_gen < 0 || n_prompt + n_gen > m->hp.n_ctx)
        return fail("qwen2: bad prompt/generation size");
    int32_t next = 0;
    for (int32_t i = 0; i < n_prompt; i++)
        if (mi_qwen2_decode(m, prompt[i], i, &next, nullptr)) return -1;
    // n_gen timed decode steps; the first one consumes the prompt's greedy continuation
    return mi_qwen2_decode_steps(m, next, n_prompt, n_gen, out_tokens, gen_seconds);
}

int mi_qwen2_get_cache_seq(mi_qwen2 *m, int32_t layer, int32_t is_v, int32_t seq, int32_t n_pos, void *dst,
                           size_t size) {
    if (check_cache_args(m, layer, seq, n_pos)) return -1;
    ggml_tensor *c = is_v ? m->v_cache[layer] : m->k_cache[layer];
    const size_t bytes = (size_t)n_pos * c->nb[1];
    if (!dst || size != bytes) return fail("qwen2: cache copy needs %zu bytes, got %zu", bytes, size);
    if (bytes) ggml_backend_tensor_get(c, dst, (size_t)seq * m->hp.n_ctx * c->nb[1], bytes);
    return 0;
}

int mi_qwen2_set_cache_seq(mi_qwen2 *m, int32_t layer, int32_t is_v, int32_t seq, int32_t n_pos, const void *src,
                           size_t size) {
    if (check_cache_args(m, layer, seq, n_pos)) return -1;
    ggml_tensor *c = is_v ? m->v_cache[layer] : m->k_cache[layer];
    const size_t bytes = (size_t)n_pos * c->nb[1];
    if (!src || size != bytes) return fail("qwen2: cache copy needs %zu bytes, got %zu", bytes, size);
    if (bytes) ggml_backend_tensor_set(c, src, (size_t)seq * m->hp.n_ctx * c->nb[1], bytes);
    return 0;
}

int mi_qwen2_get_cache(mi_qwen2 *m, int32_t layer, int32_t is_v, int32_t n_pos, void *dst, size_t size) {
    return mi_qwen2_get_cache_seq(m, layer, is_v, 0, n_pos, dst, size);
}

int mi_qwen2_persist_timing(mi_qwen2 *m, int64_t *launches, double *total_ms) {
    if (!m || !launches || !total_ms) return fail("qwen2: persist_timing: null argument");
    if (ggml_backend_mi355x_persist_timing(m->backend, launches, total_ms) != 0)
        return fail("qwen2: persistent-launch timing is off (GGML_MI355X_PERSIST_TIMING=1 at model creation)");
    return 0;
}

int mi_qwen2_fill_cache(mi_qwen2 *m, int32_t n_pos, uint64_t seed, float scale) {
    if (n_pos < 0 || n_pos > m->hp.n_ctx) return fail("qwen2: n_pos %d outside the cache", n_pos);
    for (int il = 0; il < m->hp.n_layer; il++) {
        for (int kv = 0; kv < 2; kv++) {
            ggml_tensor *c = kv ? m->v_cache[il] : m->k_cache[il];
            for (int s = 0; s < m->n_seq; s++) {
                uint8_t *base = (uint8_t *)c->data + (size_t)s * m->hp.n_ctx * c->nb[1];
                const uint64_t sd = seed + 0x1000003ull * (uint64_t)((il * 2 + kv) * m->n_seq + s);
                if (mi_fill_f16_uniform(nullptr, base, n_pos, c->ne[0], c->nb[1], sd, scale))
                    return fail("qwen2: cache fill failed: %s", mi_last_error());
            }
        }
    }
    if (mi_device_sync()) return fail("qwen2: cache fill failed: %s", mi_last_error());
    return 0;
}

}  // extern "C"

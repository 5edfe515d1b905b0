// Model drivers above the backend seam: C++ restatement of the reference's
// Llama (src/arch/llm/llama.rs) and Lfm2 (src/arch/llm/lfm2.rs) schedules,
// issuing the same backend calls in the same order through the C ABI of
// include/kernrt_hip.h, plus an on-device greedy loop.
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/kernrt_llm.h"
#include "internal.hpp"

namespace {

struct Norms {
    kr_buf att, ffn, q, k;
    bool has_q, has_k;
};

struct PrefillBuffers {
    size_t n_tok = 0;
    kr_buf x, xb, q, k, v, attn, o, bcx, h, co, cy, gate, up, att;
};

struct Row {
    size_t token, rope_pos, slot, att_start, sh_start, sh_end;
};

}  // namespace

struct krl_model {
    kr_ctx* b = nullptr;
    krl_config c{};
    bool lfm2 = false;
    std::string err;
    std::vector<bool> is_attention;
    std::vector<size_t> conv_k;
    std::vector<Norms> norms;
    std::vector<long> conv_kernels, conv_state;
    kr_buf rms_final = 0;
    kr_buf x, x2, xb, q, k, v, attn, o, bcx, h, co, cy, gate, up, mlp, hidden, att, logits;
    kr_buf batch_logits = 0;  // [rows][vocab] for decode_batch
    size_t batch_logits_rows = 0;
    std::vector<float> logits_host;
    bool has_prefill = false;
    PrefillBuffers pb;
    uint32_t* step = nullptr;  // device step record (internal.hpp)
    hipGraph_t graph = nullptr;  // one captured decode step
    hipGraphExec_t graph_exec = nullptr;
    uint64_t graph_epoch = 0;
    size_t graph_cap = 0;  // the longest window the captured step serves
    bool fused = true;  // KERNRT_HIP_UNFUSED=1 runs the reference's op-by-op schedule
};

namespace {

#define KRC(m, expr)                                          \
    do {                                                      \
        int rc_ = (expr);                                     \
        if (rc_ != KR_OK) {                                   \
            (m)->err = std::string(#expr) + ": " + kr_last_error((m)->b); \
            return rc_;                                       \
        }                                                     \
    } while (0)

int alloc(krl_model* m, size_t n, kr_buf* out) {
    KRC(m, kr_alloc(m->b, n, out));
    return KR_OK;
}

int upload(krl_model* m, const float* d, size_t n, kr_buf* out) {
    KRC(m, kr_upload(m->b, d, n, out));
    return KR_OK;
}

#define TRY(expr)                  \
    do {                           \
        int rc2_ = (expr);         \
        if (rc2_ != KR_OK) return rc2_; \
    } while (0)

// Llama::with_backend (llama.rs:364-415) / Lfm2::with_backend (lfm2.rs:276-366)
int construct(krl_model* m, const krl_weights* w) {
    const krl_config& c = m->c;
    size_t kv_dim = c.n_kv_heads * c.head_dim, q_dim = c.n_heads * c.head_dim, dim = c.dim;
    KRC(m, kr_prepare(m->b, c.n_layers, kv_dim, c.seq_len));
    const char* unfused = getenv("KERNRT_HIP_UNFUSED");
    m->fused = !(unfused && unfused[0] == '1');
    for (size_t l = 0; l < c.n_layers; l++) {
        const krl_layer& L = w->layers[l];
        Norms n{};
        TRY(upload(m, L.rms_att, dim, &n.att));
        TRY(upload(m, L.rms_ffn, dim, &n.ffn));
        n.has_q = L.rms_q != nullptr;
        n.has_k = L.rms_k != nullptr;
        if (n.has_q) TRY(upload(m, L.rms_q, c.head_dim, &n.q));
        if (n.has_k) TRY(upload(m, L.rms_k, c.head_dim, &n.k));
        m->norms.push_back(n);
    }
    TRY(upload(m, w->rms_final, dim, &m->rms_final));
    for (size_t l = 0; l < c.n_layers; l++) {
        const krl_layer& L = w->layers[l];
        m->is_attention.push_back(!m->lfm2 || L.is_attention);
        if (m->lfm2 && L.conv_kernel) {  // lfm2.rs:306-330
            size_t k = L.conv_k;
            kr_buf kb, ring, zeros;
            TRY(upload(m, L.conv_kernel, dim * k, &kb));
            size_t ring_len = dim * std::max<size_t>(k - 1, 1);
            TRY(alloc(m, ring_len, &ring));
            std::vector<float> z(ring_len, 0.0f);
            TRY(upload(m, z.data(), ring_len, &zeros));
            KRC(m, kr_copy(m->b, zeros, 0, ring, 0, ring_len));
            m->conv_kernels.push_back((long)kb);
            m->conv_state.push_back((long)ring);
            m->conv_k.push_back(k);
        } else {
            m->conv_kernels.push_back(-1);
            m->conv_state.push_back(-1);
            m->conv_k.push_back(0);
        }
    }
    TRY(alloc(m, dim, &m->x));
    TRY(alloc(m, dim, &m->x2));
    TRY(alloc(m, dim, &m->xb));
    TRY(alloc(m, q_dim, &m->q));
    TRY(alloc(m, kv_dim, &m->k));
    TRY(alloc(m, kv_dim, &m->v));
    TRY(alloc(m, q_dim, &m->attn));
    TRY(alloc(m, dim, &m->o));
    if (m->lfm2) {
        TRY(alloc(m, 3 * dim, &m->bcx));
        TRY(alloc(m, dim, &m->h));
        TRY(alloc(m, dim, &m->co));
        TRY(alloc(m, dim, &m->cy));
    }
    TRY(alloc(m, c.hidden_dim, &m->gate));
    TRY(alloc(m, c.hidden_dim, &m->up));
    TRY(alloc(m, dim, &m->mlp));
    TRY(alloc(m, dim, &m->hidden));
    TRY(alloc(m, c.n_heads * c.seq_len, &m->att));
    TRY(alloc(m, c.vocab_size, &m->logits));
    m->logits_host.assign(c.vocab_size, 0.0f);
    int rc = kri::device_u32(m->b, 8, &m->step);
    if (rc) {
        m->err = kr_last_error(m->b);
        return rc;
    }
    return KR_OK;
}

struct Geometry {
    size_t dim, hidden, q_dim, kv_dim, hs;
    float eps;
    kr_attn_spec as;
    kr_rope_spec rs;
};

Geometry geometry(const krl_config& c) {
    Geometry g;
    g.dim = c.dim;
    g.hidden = c.hidden_dim;
    g.hs = c.head_dim;
    g.q_dim = c.n_heads * c.head_dim;
    g.kv_dim = c.n_kv_heads * c.head_dim;
    g.eps = c.rms_eps;
    g.as = kr_attn_spec{c.n_heads, c.n_heads / c.n_kv_heads, c.head_dim, g.kv_dim, c.seq_len};
    g.rs = kr_rope_spec{c.head_dim, c.rope_theta, c.rope_interleaved};
    return g;
}

// The decode step with fused kernels: same values as the op-by-op schedule
// below. Each residual add_in_place is folded into the rms_norm that follows
// it, and every projection input is quantized by the kernel that produces it.
// Where the width allows, the attention and FFN norms run inside the launch
// of the projection that consumes them; the residual row then alternates
// between two buffers, because that launch's workgroups all still read the
// old row while one of them writes the new one.
// dev: the token, window and position come from the device step record, and
// `cap` bounds the window (the launches are sized for it); else from the host.
int decode_step_fused(krl_model* m, size_t token, size_t pos, bool dev, size_t cap) {
    kr_ctx* b = m->b;
    Geometry g = geometry(m->c);
    const uint32_t* s = m->step;
    const bool pro = kri::pro_fusable(g.dim) && kri::pro_fusable(g.q_dim);
    const size_t wmax = dev ? cap : pos + 1;
    const bool split = kri::split_attention_ok(b, &g.as, wmax);
    kr_buf X[2] = {m->x, m->x2};
    int cur = 0;
    if (dev)
        KRC(m, kri::embed_dev(b, s + 0, m->x, 0));
    else
        KRC(m, kr_embed(b, token, m->x, 0));
    size_t positions[1] = {pos};
    kr_window win{0, pos, 0, 0};
    kr_buf pending = KR_NO_BUF;  // the residual still to add into x
    // norm(x + add) feeding the projections projs -> ys
    auto norm_then = [&](kr_buf add, kr_buf w, size_t l, const int* projs, const kr_buf* ys, int n) -> int {
        if (pro) {
            KRC(m, kri::norm_project(b, l, projs, ys, n, X[cur], add, w, X[cur ^ 1], g.dim, g.eps));
            cur ^= 1;
        } else {
            KRC(m, kri::norm_quant(b, X[cur], add, 1, w, m->xb, 1, g.dim, g.eps));
            KRC(m, kri::project_q(b, l, projs, ys, n, 1));
        }
        return KR_OK;
    };
    for (size_t l = 0; l < m->c.n_layers; l++) {
        const Norms& n = m->norms[l];
        if (m->is_attention[l]) {
            int qkv[3] = {KR_PROJ_Q, KR_PROJ_K, KR_PROJ_V};
            kr_buf ys[3] = {m->q, m->k, m->v};
            TRY(norm_then(pending, n.att, l, qkv, ys, 3));
            if (split && pro) {
                // q/k norms + rope + kv_write + attention in two launches; O quantizes its input
                KRC(m, kri::rope_attention(b, m->q, m->k, m->v, m->attn, m->att, l, pos, dev ? s : nullptr, &g.as,
                                           &g.rs, wmax, n.has_q ? n.q : KR_NO_BUF, n.has_k ? n.k : KR_NO_BUF,
                                           g.eps));
                KRC(m, kri::quant_project(b, l, KR_PROJ_O, m->attn, m->o, g.q_dim));
            } else {
                if (n.has_q && n.has_k) {
                    KRC(m, kri::qk_norm_pair(b, m->q, m->k, 1, g.q_dim, g.kv_dim, g.hs, n.q, n.k, g.eps));
                } else {
                    if (n.has_q) KRC(m, kr_qk_norm(b, m->q, 1, g.q_dim, g.hs, n.q, g.eps));
                    if (n.has_k) KRC(m, kr_qk_norm(b, m->k, 1, g.kv_dim, g.hs, n.k, g.eps));
                }
                KRC(m, kri::rope_kv(b, m->q, m->k, m->v, g.q_dim, g.kv_dim, 1, dev ? nullptr : positions,
                                    dev ? nullptr : positions, dev ? s + 2 : nullptr, l, &g.rs));
                if (g.hs % 32 == 0) {
                    KRC(m, kri::attention_quant(b, m->q, m->attn, m->att, l, dev ? nullptr : &win, 1,
                                                dev ? s + 1 : nullptr, &g.as));
                } else {  // head outputs are not whole Q8 blocks: quantize the row after
                    if (dev)
                        KRC(m, kri::attention_dev(b, m->q, m->attn, m->att, l, s + 1, &g.as));
                    else
                        KRC(m, kr_attention(b, m->q, m->attn, m->att, l, &win, 1, &g.as));
                    KRC(m, kr_quantize_rows(b, m->attn, 1, g.q_dim));
                }
                int o[1] = {KR_PROJ_O};
                KRC(m, kri::project_q(b, l, o, &m->o, 1, 1));
            }
        } else {
            int ci[1] = {KR_PROJ_CONV_IN};
            TRY(norm_then(pending, n.att, l, ci, &m->bcx, 1));
            // B * x, the conv and C * conv in one launch; out_proj quantizes its input
            KRC(m, kri::conv_block_decode(b, m->cy, m->bcx, (kr_buf)m->conv_kernels[l], (kr_buf)m->conv_state[l],
                                          g.dim, m->conv_k[l]));
            if (pro)
                KRC(m, kri::quant_project(b, l, KR_PROJ_CONV_OUT, m->cy, m->o, g.dim));
            else
                KRC(m, kr_project(b, l, KR_PROJ_CONV_OUT, m->cy, m->o, 1));
        }
        int gu[2] = {KR_PROJ_GATE, KR_PROJ_UP};
        kr_buf gys[2] = {m->gate, m->up};
        if (pro && kri::swiglu_ok(b, l, g.dim)) {
            // gate/up, SiLU * up and its Q8 in one launch (each workgroup owns
            // 32 rows of both matrices, so no workgroup redoes another's work)
            KRC(m, kri::norm_swiglu(b, l, X[cur], m->o, n.ffn, X[cur ^ 1], m->gate, g.dim, g.eps));
            cur ^= 1;
        } else {
            TRY(norm_then(m->o, n.ffn, l, gu, gys, 2));
            KRC(m, kri::silu_quant(b, m->gate, m->up, 1, g.hidden));
        }
        // the final norm stays a separate launch: folded into the classifier,
        // 49k rows' worth of workgroups would each redo its serial sum
        int dn[1] = {KR_PROJ_DOWN};
        KRC(m, kri::project_q(b, l, dn, &m->mlp, 1, 1));
        pending = m->mlp;
    }
    KRC(m, kri::norm_quant(b, X[cur], pending, 1, m->rms_final, m->xb, 1, g.dim, g.eps));
    KRC(m, kri::logits_q(b, m->logits));
    if (dev) KRC(m, kri::greedy_step(b, m->logits, m->c.vocab_size, m->step));
    return KR_OK;
}

// One decode step, llama.rs:816-859 / lfm2.rs:414-474. With `dev`, the
// token, position and window come from the device step record.
int decode_step(krl_model* m, size_t token, size_t pos, bool dev, size_t cap) {
    if (m->fused) return decode_step_fused(m, token, pos, dev, cap);
    kr_ctx* b = m->b;
    Geometry g = geometry(m->c);
    const uint32_t* s = m->step;
    if (dev)
        KRC(m, kri::embed_dev(b, s + 0, m->x, 0));
    else
        KRC(m, kr_embed(b, token, m->x, 0));
    size_t positions[1] = {pos};
    kr_window win{0, pos, 0, 0};
    for (size_t l = 0; l < m->c.n_layers; l++) {
        const Norms& n = m->norms[l];
        KRC(m, kr_rms_norm(b, m->xb, m->x, n.att, 1, g.dim, g.eps));
        if (m->is_attention[l]) {
            KRC(m, kr_project_qkv(b, l, m->xb, m->q, m->k, m->v, 1));
            if (n.has_q) KRC(m, kr_qk_norm(b, m->q, 1, g.q_dim, g.hs, n.q, g.eps));
            if (n.has_k) KRC(m, kr_qk_norm(b, m->k, 1, g.kv_dim, g.hs, n.k, g.eps));
            if (dev) {
                KRC(m, kri::rope_dev(b, m->q, m->k, g.q_dim, g.kv_dim, s + 2, &g.rs));
                KRC(m, kri::kv_write_dev(b, l, s + 2, m->k, m->v));
                KRC(m, kri::attention_dev(b, m->q, m->attn, m->att, l, s + 1, &g.as));
            } else {
                KRC(m, kr_rope(b, m->q, m->k, g.q_dim, g.kv_dim, 1, positions, &g.rs));
                KRC(m, kr_kv_write(b, l, positions, m->k, m->v, 1));
                KRC(m, kr_attention(b, m->q, m->attn, m->att, l, &win, 1, &g.as));
            }
            KRC(m, kr_project(b, l, KR_PROJ_O, m->attn, m->o, 1));
            KRC(m, kr_add_in_place(b, m->x, m->o, g.dim));
        } else {
            KRC(m, kr_project(b, l, KR_PROJ_CONV_IN, m->xb, m->bcx, 1));
            KRC(m, kr_mul(b, m->h, 0, m->bcx, 0, m->bcx, 2 * g.dim, g.dim));
            KRC(m, kr_conv_decode(b, m->co, m->h, (kr_buf)m->conv_kernels[l], (kr_buf)m->conv_state[l], g.dim,
                                  m->conv_k[l]));
            KRC(m, kr_mul(b, m->cy, 0, m->bcx, g.dim, m->co, 0, g.dim));
            KRC(m, kr_project(b, l, KR_PROJ_CONV_OUT, m->cy, m->o, 1));
            KRC(m, kr_add_in_place(b, m->x, m->o, g.dim));
        }
        KRC(m, kr_rms_norm(b, m->xb, m->x, n.ffn, 1, g.dim, g.eps));
        KRC(m, kr_project_gate_up(b, l, m->xb, m->gate, m->up, 1));
        KRC(m, kr_silu_mul(b, m->gate, m->up, g.hidden));
        KRC(m, kr_project(b, l, KR_PROJ_DOWN, m->gate, m->mlp, 1));
        KRC(m, kr_add_in_place(b, m->x, m->mlp, g.dim));
    }
    KRC(m, kr_rms_norm(b, m->xb, m->x, m->rms_final, 1, g.dim, g.eps));
    KRC(m, kr_logits(b, m->xb, m->logits));
    if (dev) KRC(m, kri::greedy_step(b, m->logits, m->c.vocab_size, m->step));
    return KR_OK;
}

// PrefillBuffers::new (llama.rs:148-166, lfm2.rs:84-106)
int ensure_prefill(krl_model* m, size_t n_tok) {
    if (m->has_prefill && m->pb.n_tok >= n_tok) return KR_OK;
    Geometry g = geometry(m->c);
    PrefillBuffers& p = m->pb;
    p.n_tok = n_tok;
    TRY(alloc(m, n_tok * g.dim, &p.x));
    TRY(alloc(m, n_tok * g.dim, &p.xb));
    TRY(alloc(m, n_tok * g.q_dim, &p.q));
    TRY(alloc(m, n_tok * g.kv_dim, &p.k));
    TRY(alloc(m, n_tok * g.kv_dim, &p.v));
    TRY(alloc(m, n_tok * g.q_dim, &p.attn));
    TRY(alloc(m, 4 * n_tok * g.dim, &p.o));  // room for a chain-split projection's four planes
    if (m->lfm2) {
        TRY(alloc(m, n_tok * 3 * g.dim, &p.bcx));
        TRY(alloc(m, n_tok * g.dim, &p.h));
        TRY(alloc(m, n_tok * g.dim, &p.co));
        TRY(alloc(m, n_tok * g.dim, &p.cy));
    }
    TRY(alloc(m, n_tok * g.hidden, &p.gate));
    TRY(alloc(m, n_tok * g.hidden, &p.up));
    TRY(alloc(m, n_tok * m->c.n_heads * m->c.seq_len, &p.att));
    m->has_prefill = true;
    return KR_OK;
}

// The conv of an LFM2 prefill, h = p.h -> p.co, and the ring it leaves.
// Batched (lfm2.rs:587-603): zero history below the first row, then the last
// k - 1 rows of h copied into the tail of the ring. Stepped: the values the
// reference's per-token prefill of a Q8_0 model (lfm2.rs:490-495) produces,
// i.e. conv_decode row by row through the ring, in one launch plus the ring
// advance.
int prefill_conv(krl_model* m, size_t l, size_t n_tok, bool stepped) {
    kr_ctx* b = m->b;
    PrefillBuffers& p = m->pb;
    size_t dim = m->c.dim, k = m->conv_k[l];
    if (stepped) {
        KRC(m, kri::conv_prefill_stepped(b, p.co, p.h, (kr_buf)m->conv_kernels[l], (kr_buf)m->conv_state[l], n_tok,
                                         dim, k));
        return KR_OK;
    }
    KRC(m, kr_conv_prefill(b, p.co, p.h, (kr_buf)m->conv_kernels[l], n_tok, dim, k));
    if (m->conv_state[l] >= 0) {
        size_t take = std::min(n_tok, k - 1);
        KRC(m, kr_copy(b, p.h, (n_tok - take) * dim, (kr_buf)m->conv_state[l], (k - 1 - take) * dim, take * dim));
    }
    return KR_OK;
}

// llama.rs:690-771, generalised with the LFM2 conv branch of lfm2.rs:559-632.
// `stepped_conv`: the conv layers reproduce a token-by-token prefill
// (prefill_conv).
int prefill_rows(krl_model* m, const std::vector<Row>& rows, bool stepped_conv = false) {
    kr_ctx* b = m->b;
    Geometry g = geometry(m->c);
    size_t n_tok = rows.size();
    std::vector<size_t> positions, slots;
    std::vector<kr_window> windows;
    for (const Row& r : rows) {
        positions.push_back(r.rope_pos);
        slots.push_back(r.slot);
        windows.push_back(kr_window{r.att_start, r.slot, r.sh_start, r.sh_end});
    }
    TRY(ensure_prefill(m, n_tok));
    PrefillBuffers& p = m->pb;
    if (m->fused) {
        std::vector<size_t> toks(n_tok);
        for (size_t r = 0; r < n_tok; r++) toks[r] = rows[r].token;
        KRC(m, kri::embed_rows(b, toks.data(), n_tok, p.x));  // one launch for every row
    } else {
        for (size_t r = 0; r < n_tok; r++) KRC(m, kr_embed(b, rows[r].token, p.x, r * g.dim));
    }
    if (m->fused) {
        // prefill_rows with the fused kernels (see decode_step_fused); the
        // last residual add is applied here because the final norm reads one row
        // `pending` is the last projection into the residual stream, one plane
        // or a chain-split projection's four partial-sum planes
        kr_buf pending = KR_NO_BUF;
        int planes = 1;
        for (size_t l = 0; l < m->c.n_layers; l++) {
            const Norms& n = m->norms[l];
            KRC(m, kri::norm_quant(b, p.x, pending, planes, n.att, p.xb, n_tok, g.dim, g.eps));
            if (m->is_attention[l]) {
                if (!n.has_q && !n.has_k && kri::qkv_rope_ok(b, l, n_tok, &g.rs)) {
                    // one launch: q/k/v, RoPE and kv_write
                    KRC(m, kri::project_qkv_rope(b, l, p.q, n_tok, positions.data(), slots.data(), &g.rs));
                } else {
                    int qkv[3] = {KR_PROJ_Q, KR_PROJ_K, KR_PROJ_V};
                    kr_buf ys[3] = {p.q, p.k, p.v};
                    KRC(m, kri::project_q(b, l, qkv, ys, 3, n_tok));
                    if (n.has_q && n.has_k && g.hs <= 128 && g.hs % 4 == 0) {
                        // q/k norms, RoPE and kv_write in one launch
                        KRC(m, kri::rope_kv(b, p.q, p.k, p.v, g.q_dim, g.kv_dim, n_tok, positions.data(),
                                            slots.data(), nullptr, l, &g.rs, n.q, n.k, g.eps));
                    } else {
                        if (n.has_q && n.has_k) {
                            KRC(m, kri::qk_norm_pair(b, p.q, p.k, n_tok, g.q_dim, g.kv_dim, g.hs, n.q, n.k, g.eps));
                        } else {
                            if (n.has_q) KRC(m, kr_qk_norm(b, p.q, n_tok, g.q_dim, g.hs, n.q, g.eps));
                            if (n.has_k) KRC(m, kr_qk_norm(b, p.k, n_tok, g.kv_dim, g.hs, n.k, g.eps));
                        }
                        KRC(m, kri::rope_kv(b, p.q, p.k, p.v, g.q_dim, g.kv_dim, n_tok, positions.data(),
                                            slots.data(), nullptr, l, &g.rs));
                    }
                }
                if (g.hs % 32 == 0) {
                    // the probabilities in p.att are scratch here: not written back
                    KRC(m, kri::attention_quant(b, p.q, p.attn, p.att, l, windows.data(), windows.size(), nullptr,
                                                &g.as, false));
                } else {
                    KRC(m, kr_attention(b, p.q, p.attn, p.att, l, windows.data(), windows.size(), &g.as));
                    KRC(m, kr_quantize_rows(b, p.attn, n_tok, g.q_dim));
                }
                int o[1] = {KR_PROJ_O};
                KRC(m, kri::project_q(b, l, o, &p.o, 1, n_tok));
            } else {
                int ci[1] = {KR_PROJ_CONV_IN};
                KRC(m, kri::project_q(b, l, ci, &p.bcx, 1, n_tok));
                // the per-row B * x products (lfm2.rs:584-595), all rows in one launch
                KRC(m, kri::mul_rows(b, p.h, 0, g.dim, p.bcx, 0, 3 * g.dim, p.bcx, 2 * g.dim, 3 * g.dim, n_tok, g.dim));
                TRY(prefill_conv(m, l, n_tok, stepped_conv));
                // the per-row C * conv_out products (lfm2.rs:611-622), all rows in one launch
                KRC(m, kri::mul_rows(b, p.cy, 0, g.dim, p.bcx, g.dim, 3 * g.dim, p.co, 0, g.dim, n_tok, g.dim));
                KRC(m, kr_project(b, l, KR_PROJ_CONV_OUT, p.cy, p.o, n_tok));
            }
            KRC(m, kri::norm_quant(b, p.x, p.o, 1, n.ffn, p.xb, n_tok, g.dim, g.eps));
            planes = 1;
            if (kri::ffn_swiglu_ok(b, l, n_tok)) {
                KRC(m, kri::ffn_swiglu_down(b, l, n_tok, p.o, 4, &planes));
            } else {
                int gu[2] = {KR_PROJ_GATE, KR_PROJ_UP};
                kr_buf gys[2] = {p.gate, p.up};
                KRC(m, kri::project_q(b, l, gu, gys, 2, n_tok));
                KRC(m, kri::silu_quant(b, p.gate, p.up, n_tok, g.hidden));
                int dn[1] = {KR_PROJ_DOWN};
                KRC(m, kri::project_q(b, l, dn, &p.o, 1, n_tok));
            }
            pending = p.o;
        }
        if (planes == 4)
            KRC(m, kri::add_planes(b, p.x, pending, n_tok * g.dim));
        else
            KRC(m, kr_add_in_place(b, p.x, pending, n_tok * g.dim));
        return KR_OK;
    }
    for (size_t l = 0; l < m->c.n_layers; l++) {
        const Norms& n = m->norms[l];
        KRC(m, kr_rms_norm(b, p.xb, p.x, n.att, n_tok, g.dim, g.eps));
        if (m->is_attention[l]) {
            KRC(m, kr_project_qkv(b, l, p.xb, p.q, p.k, p.v, n_tok));
            if (n.has_q) KRC(m, kr_qk_norm(b, p.q, n_tok, g.q_dim, g.hs, n.q, g.eps));
            if (n.has_k) KRC(m, kr_qk_norm(b, p.k, n_tok, g.kv_dim, g.hs, n.k, g.eps));
            KRC(m, kr_rope(b, p.q, p.k, g.q_dim, g.kv_dim, n_tok, positions.data(), &g.rs));
            KRC(m, kr_kv_write(b, l, slots.data(), p.k, p.v, n_tok));
            KRC(m, kr_attention(b, p.q, p.attn, p.att, l, windows.data(), windows.size(), &g.as));
            KRC(m, kr_project(b, l, KR_PROJ_O, p.attn, p.o, n_tok));
            KRC(m, kr_add_in_place(b, p.x, p.o, n_tok * g.dim));
        } else {
            KRC(m, kr_project(b, l, KR_PROJ_CONV_IN, p.xb, p.bcx, n_tok));
            for (size_t r = 0; r < n_tok; r++)
                KRC(m, kr_mul(b, p.h, r * g.dim, p.bcx, r * 3 * g.dim, p.bcx, r * 3 * g.dim + 2 * g.dim, g.dim));
            TRY(prefill_conv(m, l, n_tok, stepped_conv));
            for (size_t r = 0; r < n_tok; r++)
                KRC(m, kr_mul(b, p.cy, r * g.dim, p.bcx, r * 3 * g.dim + g.dim, p.co, r * g.dim, g.dim));
            KRC(m, kr_project(b, l, KR_PROJ_CONV_OUT, p.cy, p.o, n_tok));
            KRC(m, kr_add_in_place(b, p.x, p.o, n_tok * g.dim));
        }
        KRC(m, kr_rms_norm(b, p.xb, p.x, n.ffn, n_tok, g.dim, g.eps));
        KRC(m, kr_project_gate_up(b, l, p.xb, p.gate, p.up, n_tok));
        KRC(m, kr_silu_mul(b, p.gate, p.up, n_tok * g.hidden));
        KRC(m, kr_project(b, l, KR_PROJ_DOWN, p.gate, p.o, n_tok));
        KRC(m, kr_add_in_place(b, p.x, p.o, n_tok * g.dim));
    }
    return KR_OK;
}

// llama.rs:652-683
int final_hiddens(krl_model* m, const std::vector<long>& rows, float* out) {
    size_t dim = m->c.dim;
    for (size_t i = 0; i < rows.size(); i++) {
        if (rows[i] < 0) {
            memset(out + i * dim, 0, dim * sizeof(float));
            continue;
        }
        KRC(m, kr_copy(m->b, m->pb.x, (size_t)rows[i] * dim, m->hidden, 0, dim));
        KRC(m, kr_rms_norm(m->b, m->xb, m->hidden, m->rms_final, 1, dim, m->c.rms_eps));
        KRC(m, kr_read(m->b, m->xb, out + i * dim, dim));
    }
    return KR_OK;
}

int fail(krl_model* m, const char* msg) {
    m->err = msg;
    return KR_ERR_INVALID;
}

int make(kr_ctx* backend, const krl_config* cfg, const krl_weights* w, bool lfm2, krl_model** out) {
    *out = nullptr;
    if (!backend || !cfg || !w || !w->layers || !w->rms_final) return KR_ERR_INVALID;
    if (cfg->n_kv_heads == 0 || cfg->n_heads % cfg->n_kv_heads != 0 || cfg->head_dim == 0)
        return KR_ERR_INVALID;
    krl_model* m = new krl_model();
    m->b = backend;
    m->c = *cfg;
    m->lfm2 = lfm2;
    int rc = construct(m, w);
    if (rc != KR_OK) {
        kri::set_error(backend, rc, m->err.c_str());
        krl_free(m);
        return rc;
    }
    *out = m;
    return KR_OK;
}

int drop_graph(krl_model* m) {
    if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->graph_exec = nullptr;
    m->graph = nullptr;
    return KR_OK;
}

// Capture one device-driven decode step as a graph for windows of up to
// `cap` positions (kept until the backend moves a buffer the captured kernels
// reference, or a generation needs a longer window).
int capture_step(krl_model* m, size_t cap) {
    hipStream_t st = kri::stream(m->b);
    drop_graph(m);
    if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess)
        return fail(m, "graph capture could not start");
    int rc = decode_step(m, 0, 0, true, cap);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(st, &graph);
    if (rc != KR_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess || hipGraphInstantiate(&m->graph_exec, graph, nullptr, nullptr, 0) != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        m->graph_exec = nullptr;
        return fail(m, "graph instantiation failed");
    }
    m->graph = graph;
    m->graph_epoch = kri::epoch(m->b);
    m->graph_cap = cap;
    return KR_OK;
}

}  // namespace

extern "C" {

int krl_llama_new(kr_ctx* backend, const krl_config* cfg, const krl_weights* w, krl_model** out) {
    return make(backend, cfg, w, false, out);
}

int krl_lfm2_new(kr_ctx* backend, const krl_config* cfg, const krl_weights* w, krl_model** out) {
    return make(backend, cfg, w, true, out);
}

void krl_free(krl_model* m) {
    if (!m) return;
    drop_graph(m);
    if (m->step) {
        kr_synchronize(m->b);
        kri::device_free(m->step);
    }
    delete m;
}

const char* krl_last_error(const krl_model* m) { return m ? m->err.c_str() : "no model"; }

int krl_forward(krl_model* m, size_t token, size_t pos, float* logits) {
    if (pos >= m->c.seq_len) return fail(m, "position past the context length");
    TRY(decode_step(m, token, pos, false, pos + 1));
    KRC(m, kr_read(m->b, m->logits, logits, m->c.vocab_size));
    return KR_OK;
}

// llama.rs:473-536 / lfm2.rs:481-640. Every storage runs batched. Where the
// reference loops forward() per token instead (storages other than f32, bf16
// and q8_0x4: here q8_0), the batch reproduces that loop's values: for Llama
// the rows are independent apart from causal attention, which reads the same
// cache either way; for LFM2 the conv layers take their history from the ring
// (prefill_conv's stepped form) instead of zero padding.
int krl_prefill(krl_model* m, const size_t* tokens, size_t n, size_t start, float* logits) {
    if (start + n > m->c.seq_len) return fail(m, "prefill runs past the context length");
    if (n == 0) {
        memcpy(logits, m->logits_host.data(), m->c.vocab_size * sizeof(float));
        return KR_OK;
    }
    std::vector<Row> rows;
    for (size_t i = 0; i < n; i++) rows.push_back(Row{tokens[i], start + i, start + i, 0, 0, 0});
    const char* storage = kr_storage(m->b);
    bool batched_in_reference =
        !strcmp(storage, "f32") || !strcmp(storage, "bf16") || !strcmp(storage, "q8_0x4");  // lfm2.rs:489
    TRY(prefill_rows(m, rows, m->lfm2 && !batched_in_reference));
    size_t dim = m->c.dim;
    KRC(m, kr_copy(m->b, m->pb.x, (n - 1) * dim, m->hidden, 0, dim));
    KRC(m, kr_rms_norm(m->b, m->xb, m->hidden, m->rms_final, 1, dim, m->c.rms_eps));
    KRC(m, kr_logits(m->b, m->xb, m->logits));
    KRC(m, kr_read(m->b, m->logits, m->logits_host.data(), m->c.vocab_size));
    memcpy(logits, m->logits_host.data(), m->c.vocab_size * sizeof(float));
    return KR_OK;
}

int krl_decode_batch(krl_model* m, const size_t* tokens, const size_t* rope_pos, const size_t* slots,
                     const size_t* att_start, size_t n_seq, float* logits) {
    if (m->lfm2) return fail(m, "decode_batch is a Llama entry point");
    if (n_seq == 0) return KR_OK;
    std::vector<Row> rows;
    for (size_t s = 0; s < n_seq; s++) {
        if (slots[s] >= m->c.seq_len || att_start[s] > slots[s]) return fail(m, "decode_batch row out of range");
        rows.push_back(Row{tokens[s], rope_pos[s], slots[s], att_start[s], 0, 0});
    }
    TRY(prefill_rows(m, rows));
    // the final norm and the classifier over every row (cpu.rs:501-514 per row)
    const size_t vocab = m->c.vocab_size, dim = m->c.dim;
    if (m->batch_logits_rows < n_seq) {
        TRY(alloc(m, n_seq * vocab, &m->batch_logits));
        m->batch_logits_rows = n_seq;
    }
    KRC(m, kri::norm_quant(m->b, m->pb.x, KR_NO_BUF, 1, m->rms_final, m->pb.xb, n_seq, dim, m->c.rms_eps));
    KRC(m, kri::logits_rows(m->b, m->batch_logits, n_seq));
    if (logits) KRC(m, kr_read(m->b, m->batch_logits, logits, n_seq * vocab));
    return KR_OK;
}

// llama.rs:552-580
int krl_prefill_multi(krl_model* m, const size_t* tokens, const size_t* lens, size_t n_seq, float* hiddens) {
    if (m->lfm2) return fail(m, "prefill_multi is a Llama entry point");
    std::vector<Row> rows;
    std::vector<long> last;
    size_t offset = 0, at = 0;
    for (size_t s = 0; s < n_seq; s++) {
        if (lens[s] == 0) {
            last.push_back(-1);
            continue;
        }
        if (offset + lens[s] > m->c.seq_len) return fail(m, "prefill_multi runs past the context length");
        for (size_t i = 0; i < lens[s]; i++) rows.push_back(Row{tokens[at + i], i, offset + i, offset, 0, 0});
        at += lens[s];
        last.push_back((long)rows.size() - 1);
        offset += lens[s];
    }
    if (!rows.empty()) TRY(prefill_rows(m, rows));
    return final_hiddens(m, last, hiddens);
}

// llama.rs:603-647
int krl_prefill_shared(krl_model* m, const size_t* prefix, size_t n_prefix, const size_t* tokens,
                       const size_t* lens, size_t n_seq, float* hiddens) {
    if (m->lfm2) return fail(m, "prefill_shared is a Llama entry point");
    if (n_prefix > m->c.seq_len) return fail(m, "prefill_shared prefix runs past the context length");
    std::vector<Row> rows;
    for (size_t i = 0; i < n_prefix; i++) rows.push_back(Row{prefix[i], i, i, 0, 0, 0});
    std::vector<long> last;
    size_t base = n_prefix, at = 0;
    for (size_t s = 0; s < n_seq; s++) {
        if (lens[s] == 0) {
            last.push_back(-1);
            continue;
        }
        if (base + lens[s] > m->c.seq_len) return fail(m, "prefill_shared runs past the context length");
        for (size_t i = 0; i < lens[s]; i++)
            rows.push_back(Row{tokens[at + i], n_prefix + i, base + i, base, 0, n_prefix});
        at += lens[s];
        last.push_back((long)rows.size() - 1);
        base += lens[s];
    }
    if (!rows.empty()) TRY(prefill_rows(m, rows));
    return final_hiddens(m, last, hiddens);
}

int krl_generate_greedy(krl_model* m, size_t token, size_t pos, size_t n_steps, size_t* out_tokens, int use_graph) {
    if (n_steps == 0) return KR_OK;
    if (pos + n_steps > m->c.seq_len) return fail(m, "generation runs past the context length");
    if (n_steps > kri::token_ring_len()) return fail(m, "too many steps for the token ring");
    if (token >= m->c.vocab_size) return fail(m, "token out of range");
    hipStream_t st = kri::stream(m->b);
    uint32_t init[8] = {(uint32_t)token, 0, (uint32_t)pos, 0, 0, 0, 0, 0};
    if (hipMemcpyAsync(m->step, init, sizeof init, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fail(m, "step record upload failed");
    // the window bucket: the smallest power of two from 512 covering the
    // last step's window (pos + n_steps positions), at most the context, so
    // that short generations on a long context take the split attention
    const size_t need = pos + n_steps;
    size_t cap = 512;
    while (cap < need) cap *= 2;
    cap = std::min(cap, (size_t)m->c.seq_len);
    size_t i = 0;
    if (use_graph) {
        // The first step runs eagerly when no valid graph exists: it performs
        // every lazy allocation, so the capture records kernels only. A graph
        // captured for a shorter window is replaced.
        if (!m->graph_exec || m->graph_epoch != kri::epoch(m->b) || m->graph_cap < need) {
            TRY(decode_step(m, 0, 0, true, cap));
            i = 1;
            if (n_steps > 1) TRY(capture_step(m, cap));
        }
        hipError_t e = hipSuccess;
        for (; i < n_steps && e == hipSuccess; i++) e = hipGraphLaunch(m->graph_exec, st);
        if (e != hipSuccess) return fail(m, "graph launch failed");
    } else {
        for (; i < n_steps; i++) TRY(decode_step(m, 0, 0, true, cap));
    }
    KRC(m, kr_read_tokens(m->b, out_tokens, n_steps));
    return KR_OK;
}

}  // extern "C"

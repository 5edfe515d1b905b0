// TEST INFRASTRUCTURE ONLY: a C ABI over the oracle so pytest (ctypes) can
// drive it. Nothing in kernrt_amd/ links or loads this library.
#include <cmath>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>

#include "oracle.hpp"

using namespace oracle;

namespace {
thread_local std::string g_err;

template <class F>
int guard(F f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

struct OWeights {
    std::shared_ptr<ModelWeights> w = std::make_shared<ModelWeights>();
};

struct OBackend {
    std::unique_ptr<Backend> b;
};

struct OModel {
    std::unique_ptr<Llama> llama;
    std::unique_ptr<Lfm2> lfm2;
};
}  // namespace

extern "C" {

struct or_config {
    size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
    float rms_eps, rope_theta;
    int rope_interleaved;
    size_t head_dim;
};

struct or_window {
    size_t att_start, slot, shared_start, shared_end;
};

const char* or_last_error() { return g_err.c_str(); }

uint16_t or_f32_to_f16_bits(float v) { return f32_to_f16_bits(v); }
float or_f16_scale_to_f32(uint16_t b) { return f16_scale_to_f32(b); }
float or_expf(float x) { return std::exp(x); }

// Q8Vec::quantize (quant.rs:831-851). `quants` holds ceil(n/32)*32 values.
void or_quantize(const float* x, size_t n, int8_t* quants, float* scales, uint16_t* scales_f16) {
    Q8Vec q = Q8Vec::quantize(x, n);
    std::memcpy(quants, q.quants.data(), q.quants.size());
    std::memcpy(scales, q.scales.data(), q.scales.size() * sizeof(float));
    std::memcpy(scales_f16, q.scales_f16.data(), q.scales_f16.size() * sizeof(uint16_t));
}

float or_dot_q8_0_scalar(const int8_t* a, const float* as, const int8_t* b, const float* bs,
                         size_t blocks) {
    return dot_q8_0_scalar(a, as, b, bs, blocks);
}
float or_dot_scalar(const float* a, const float* b, size_t n) { return dot_scalar(a, b, n); }
size_t or_argmax(const float* v, size_t n) { return argmax(v, n); }
void or_lcg_fill(size_t count, uint64_t seed, float* out) {
    std::vector<float> v = lcg_fill(count, seed);
    std::memcpy(out, v.data(), count * sizeof(float));
}
void or_softmax(float* x, size_t n) { softmax_in_place(x, n); }

// kind: 0 f32, 1 bf16, 2 q8_0, 3 q8_0x4 (the `cast` of tests/backends.rs:69-74)
int or_matrix_from_f32(const float* data, size_t out, size_t in, int kind, void** handle) {
    return guard([&] {
        std::vector<float> v(data, data + out * in);
        Matrix* m = new Matrix();
        bool ok = true;
        switch (kind) {
            case 0: *m = Matrix::from_f32(std::move(v), out, in); break;
            case 1: {
                Matrix f = Matrix::from_f32(std::move(v), out, in);
                *m = Matrix::from_bf16_bits(f.to_bf16_bits(), out, in);
                break;
            }
            case 2: ok = Matrix::from_f32_q8_0(v, out, in, m); break;
            case 3: ok = Matrix::from_f32_q8_0x4(v, out, in, m); break;
            default: ok = false;
        }
        if (!ok) {
            delete m;
            throw std::runtime_error("matrix shape is not valid for this storage");
        }
        *handle = m;
    });
}

// Matrices straight from quantized bytes (the `Matrix::Q8_0` fields, or
// Q8Block4 records), for tests that need blocks no f32 input produces.
int or_matrix_from_q8_0(const int8_t* quants, const float* scales, size_t out, size_t in, void** handle) {
    return guard([&] {
        if (in % Q8_0_BLOCK != 0) throw std::runtime_error("in_dim must be a multiple of 32");
        Matrix* m = new Matrix();
        m->kind = Matrix::Q8_0;
        m->out_dim = out;
        m->in_dim = in;
        m->quants.assign(quants, quants + out * in);
        m->scales.assign(scales, scales + out * in / Q8_0_BLOCK);
        *handle = m;
    });
}

int or_matrix_from_q8_0x4_blocks(const void* blocks, size_t out, size_t in, void** handle) {
    return guard([&] {
        if (in % Q8_0_BLOCK != 0 || out % 4 != 0) throw std::runtime_error("bad Q8_0x4 shape");
        Matrix* m = new Matrix();
        m->kind = Matrix::Q8_0X4;
        m->out_dim = out;
        m->in_dim = in;
        size_t n = (out / 4) * (in / Q8_0_BLOCK);
        m->blocks.resize(n);
        std::memcpy(m->blocks.data(), blocks, n * sizeof(Q8Block4));
        *handle = m;
    });
}

void or_matrix_free(void* h) { delete (Matrix*)h; }

void or_matrix_info(void* h, int* kind, size_t* out, size_t* in) {
    Matrix* m = (Matrix*)h;
    *kind = (int)m->kind;
    *out = m->out_dim;
    *in = m->in_dim;
}

void or_matrix_decode_row(void* h, size_t row, float* out) { ((Matrix*)h)->decode_row(row, out); }

int or_matrix_q8_0_data(void* h, int8_t* quants, float* scales) {
    return guard([&] {
        Matrix* m = (Matrix*)h;
        if (m->kind != Matrix::Q8_0) throw std::runtime_error("not q8_0");
        std::memcpy(quants, m->quants.data(), m->quants.size());
        std::memcpy(scales, m->scales.data(), m->scales.size() * sizeof(float));
    });
}

int or_matrix_q8_0x4_blocks(void* h, void* out) {
    return guard([&] {
        Matrix* m = (Matrix*)h;
        if (m->kind != Matrix::Q8_0X4) throw std::runtime_error("not q8_0x4");
        std::memcpy(out, m->blocks.data(), m->blocks.size() * sizeof(Q8Block4));
    });
}

int or_matrix_to_row_major(void* h, int8_t* q, float* s) {
    return guard([&] {
        std::vector<int8_t> qq;
        std::vector<float> ss;
        ((Matrix*)h)->to_row_major(&qq, &ss);
        std::memcpy(q, qq.data(), qq.size());
        std::memcpy(s, ss.data(), ss.size() * sizeof(float));
    });
}

void or_gemv_into(void* h, const float* x, float* y) { gemv_into(*(Matrix*)h, x, y); }

// Cpu::project (cpu.rs:304-371, prefill_f32 off) for one matrix, no model.
int or_project_cpu(void* h, const float* x, size_t rows, float* y) {
    return guard([&] {
        const Matrix& w = *(Matrix*)h;
        size_t in = w.in_dim, out = w.out_dim;
        if (w.kind == Matrix::Q8_0X4) {
            size_t blocks = in / Q8_0_BLOCK;
            std::vector<int8_t> bq(rows * in);
            std::vector<uint16_t> bs(rows * blocks);
            Q8Vec q8;
            for (size_t r = 0; r < rows; r++) {  // cpu.rs:143-158
                q8.quantize_into(x + r * in, in);
                std::memcpy(&bq[r * in], q8.quants.data(), in);
                std::memcpy(&bs[r * blocks], q8.scales_f16.data(), blocks * 2);
            }
            gemm_q8_0x4_batched_into(w, bq.data(), bs.data(), rows, y);
            return;
        }
        Q8Vec q8;
        for (size_t r = 0; r < rows; r++) {
            if (w.kind == Matrix::Q8_0) {
                q8.quantize_into(x + r * in, in);
                if (!gemv_q8_0_into(w, q8, y + r * out)) throw std::runtime_error("shape");
            } else {
                gemv_into(w, x + r * in, y + r * out);
            }
        }
    });
}

// Cpu::logits (cpu.rs:501-514) with an `n_x`-long input buffer.
int or_logits_cpu(void* h, const float* x, size_t n_x, float* y) {
    return guard([&] {
        const Matrix& w = *(Matrix*)h;
        if (w.kind == Matrix::Q8_0 || w.kind == Matrix::Q8_0X4) {
            Q8Vec q8;
            q8.quantize_into(x, n_x);
            if (!gemv_q8_0_into(w, q8, y)) throw std::runtime_error("shape");
        } else {
            gemv_into(w, x, y);
        }
    });
}

// Per-block exact integer dots of the weight rows (de-interleaved) with
// `rows` activation rows already quantized: out[rows][out_dim][in_dim/32].
int or_block_dots(void* h, const int8_t* xq, size_t rows, int32_t* out) {
    return guard([&] {
        const Matrix& w = *(Matrix*)h;
        std::vector<int8_t> q;
        std::vector<float> s;
        w.to_row_major(&q, &s);
        size_t in = w.in_dim, n = w.out_dim, nb = in / 32;
        for (size_t r = 0; r < rows; r++)
            for (size_t o = 0; o < n; o++)
                for (size_t b = 0; b < nb; b++) {
                    int64_t acc = 0;
                    for (size_t i = 0; i < 32; i++)
                        acc += (int64_t)q[o * in + b * 32 + i] * (int64_t)xq[r * in + b * 32 + i];
                    out[(r * n + o) * nb + b] = (int32_t)acc;
                }
    });
}

// ---- model weights ---------------------------------------------------------

void* or_weights_new(size_t n_layers) {
    OWeights* w = new OWeights();
    w->w->layers.resize(n_layers);
    return w;
}
void or_weights_free(void* w) { delete (OWeights*)w; }

void or_weights_set_embedding(void* w, void* m) { ((OWeights*)w)->w->token_embedding = *(Matrix*)m; }
void or_weights_set_classifier(void* w, void* m) {
    ((OWeights*)w)->w->wcls.reset(m ? new Matrix(*(Matrix*)m) : nullptr);
}
// proj: the Proj::index order of mod.rs:100-112
int or_weights_set_proj(void* w, size_t layer, int proj, void* m) {
    return guard([&] {
        LayerWeights& l = ((OWeights*)w)->w->layers.at(layer);
        Matrix mm = *(Matrix*)m;
        switch (proj) {
            case 0: l.wq.reset(new Matrix(mm)); break;
            case 1: l.wk.reset(new Matrix(mm)); break;
            case 2: l.wv.reset(new Matrix(mm)); break;
            case 3: l.wo.reset(new Matrix(mm)); break;
            case 4: l.w1 = mm; break;
            case 5: l.w2 = mm; break;
            case 6: l.w3 = mm; break;
            case 7: l.conv_in.reset(new Matrix(mm)); break;
            case 8: l.conv_out.reset(new Matrix(mm)); break;
            default: throw std::runtime_error("bad proj");
        }
    });
}
// which: 0 att/operator norm, 1 ffn norm, 2 q norm, 3 k norm
void or_weights_set_norm(void* w, size_t layer, int which, const float* d, size_t n) {
    LayerWeights& l = ((OWeights*)w)->w->layers.at(layer);
    std::vector<float> v(d, d + n);
    if (which == 0) l.rms_att = v;
    else if (which == 1) l.rms_ffn = v;
    else if (which == 2) l.rms_q = v;
    else l.rms_k = v;
}
void or_weights_set_final_norm(void* w, const float* d, size_t n) {
    ((OWeights*)w)->w->rms_final.assign(d, d + n);
}
void or_weights_set_conv(void* w, size_t layer, const float* kernel, size_t dim, size_t k) {
    LayerWeights& l = ((OWeights*)w)->w->layers.at(layer);
    l.conv_kernel.assign(kernel, kernel + dim * k);
    l.conv_k = k;
    l.is_attention = false;
}

static Config to_config(const or_config* c) {
    return Config{c->dim,     c->hidden_dim, c->n_layers,   c->n_heads,
                  c->n_kv_heads, c->vocab_size, c->seq_len, c->rms_eps,
                  c->rope_theta, c->rope_interleaved != 0, c->head_dim};
}

static std::unique_ptr<Backend> backend_by_name(const char* name) {
    std::string n = name;
    if (n == "cpu") return make_cpu();
    if (n == "reference") return make_reference();
    throw std::runtime_error("unknown oracle backend " + n);
}

int or_llama_new(const or_config* c, void* w, const char* backend, void** out) {
    return guard([&] {
        OModel* m = new OModel();
        m->llama.reset(new Llama(to_config(c), ((OWeights*)w)->w, backend_by_name(backend)));
        *out = m;
    });
}

int or_lfm2_new(const or_config* c, const int* is_attention, void* w, const char* backend,
                void** out) {
    return guard([&] {
        std::vector<bool> mask;
        for (size_t i = 0; i < c->n_layers; i++) mask.push_back(is_attention[i] != 0);
        OModel* m = new OModel();
        m->lfm2.reset(new Lfm2(to_config(c), mask, ((OWeights*)w)->w, backend_by_name(backend)));
        *out = m;
    });
}

void or_model_free(void* m) { delete (OModel*)m; }

int or_model_kv_fill(void* mp, size_t slots, uint64_t seed) {
    return guard([&] {
        OModel* m = (OModel*)mp;
        fill_kv(m->llama ? m->llama->backend() : m->lfm2->backend(), slots, seed);
    });
}

int or_model_kv_upload(void* mp, int which, size_t offset, const float* data, size_t len) {
    return guard([&] {
        OModel* m = (OModel*)mp;
        set_kv(m->llama ? m->llama->backend() : m->lfm2->backend(), which, offset, data, len);
    });
}

int or_model_forward(void* mp, size_t token, size_t pos, float* logits, size_t n) {
    return guard([&] {
        OModel* m = (OModel*)mp;
        const std::vector<float>& l = m->llama ? m->llama->forward(token, pos) : m->lfm2->forward(token, pos);
        std::memcpy(logits, l.data(), std::min(n, l.size()) * sizeof(float));
    });
}

int or_model_prefill(void* mp, const size_t* tokens, size_t count, size_t start, float* logits,
                     size_t n) {
    return guard([&] {
        OModel* m = (OModel*)mp;
        const std::vector<float>& l =
            m->llama ? m->llama->prefill(tokens, count, start) : m->lfm2->prefill(tokens, count, start);
        std::memcpy(logits, l.data(), std::min(n, l.size()) * sizeof(float));
    });
}

// Sequences are passed flattened: `lens[i]` tokens each, concatenated.
int or_llama_prefill_multi(void* mp, const size_t* tokens, const size_t* lens, size_t n_seq,
                           float* hiddens, size_t dim) {
    return guard([&] {
        std::vector<std::vector<size_t>> seqs;
        size_t at = 0;
        for (size_t i = 0; i < n_seq; i++) {
            seqs.emplace_back(tokens + at, tokens + at + lens[i]);
            at += lens[i];
        }
        auto h = ((OModel*)mp)->llama->prefill_multi(seqs);
        for (size_t i = 0; i < h.size(); i++) std::memcpy(hiddens + i * dim, h[i].data(), dim * sizeof(float));
    });
}

int or_llama_prefill_shared(void* mp, const size_t* prefix, size_t n_prefix, const size_t* tokens,
                            const size_t* lens, size_t n_seq, float* hiddens, size_t dim) {
    return guard([&] {
        std::vector<size_t> p(prefix, prefix + n_prefix);
        std::vector<std::vector<size_t>> seqs;
        size_t at = 0;
        for (size_t i = 0; i < n_seq; i++) {
            seqs.emplace_back(tokens + at, tokens + at + lens[i]);
            at += lens[i];
        }
        auto h = ((OModel*)mp)->llama->prefill_shared(p, seqs);
        for (size_t i = 0; i < h.size(); i++) std::memcpy(hiddens + i * dim, h[i].data(), dim * sizeof(float));
    });
}

// ---- a bare backend, for op-level checks -------------------------------------

int or_backend_new(const char* name, void* weights, size_t n_layers, size_t kv_dim, size_t seq_len,
                   void** out) {
    return guard([&] {
        OBackend* b = new OBackend();
        b->b = backend_by_name(name);
        std::shared_ptr<const ModelWeights> w =
            weights ? std::shared_ptr<const ModelWeights>(((OWeights*)weights)->w)
                    : std::make_shared<const ModelWeights>();
        b->b->prepare(w, KvSpec{n_layers, kv_dim, seq_len});
        *out = b;
    });
}
void or_backend_free(void* b) { delete (OBackend*)b; }

#define B (((OBackend*)bp)->b)
size_t or_b_alloc(void* bp, size_t len) { return B->alloc(len); }
size_t or_b_upload(void* bp, const float* d, size_t len) { return B->upload(d, len); }
void or_b_read(void* bp, size_t buf, float* out, size_t len) { B->read(buf, out, len); }
int or_b_embed(void* bp, size_t token, size_t out, size_t offset) {
    return guard([&] { B->embed(token, out, offset); });
}
void or_b_copy(void* bp, size_t s, size_t so, size_t d, size_t doff, size_t len) { B->copy(s, so, d, doff, len); }
void or_b_rms_norm(void* bp, size_t out, size_t x, size_t w, size_t rows, size_t dim, float eps) {
    B->rms_norm(out, x, w, rows, dim, eps);
}
void or_b_qk_norm(void* bp, size_t v, size_t rows, size_t width, size_t head, size_t w, float eps) {
    B->qk_norm(v, rows, width, head, w, eps);
}
void or_b_rope(void* bp, size_t q, size_t k, size_t qw, size_t kvw, size_t rows, const size_t* pos,
               size_t head_size, float theta, int interleaved) {
    B->rope(q, k, qw, kvw, rows, pos, RopeSpec{head_size, theta, interleaved != 0});
}
int or_b_project(void* bp, size_t layer, int proj, size_t x, size_t y, size_t rows) {
    return guard([&] { B->project(layer, (Proj)proj, x, y, rows); });
}
void or_b_kv_write(void* bp, size_t layer, const size_t* slots, size_t k, size_t v, size_t rows) {
    B->kv_write(layer, slots, k, v, rows);
}
void or_b_attention(void* bp, size_t q, size_t out, size_t att, size_t layer, const or_window* w,
                    size_t n, size_t n_heads, size_t kv_mul, size_t head_size, size_t kv_dim,
                    size_t seq_len) {
    std::vector<Window> ws;
    for (size_t i = 0; i < n; i++) ws.push_back({w[i].att_start, w[i].slot, w[i].shared_start, w[i].shared_end});
    B->attention(q, out, att, layer, ws.data(), n, AttnSpec{n_heads, kv_mul, head_size, kv_dim, seq_len});
}
void or_b_add_in_place(void* bp, size_t d, size_t s, size_t len) { B->add_in_place(d, s, len); }
void or_b_mul(void* bp, size_t o, size_t oo, size_t a, size_t ao, size_t b, size_t bo, size_t len) {
    B->mul(o, oo, a, ao, b, bo, len);
}
void or_b_conv_prefill(void* bp, size_t o, size_t x, size_t kern, size_t rows, size_t dim, size_t k) {
    B->conv_prefill(o, x, kern, rows, dim, k);
}
void or_b_conv_decode(void* bp, size_t o, size_t x, size_t kern, size_t state, size_t dim, size_t k) {
    B->conv_decode(o, x, kern, state, dim, k);
}
void or_b_silu_mul(void* bp, size_t g, size_t u, size_t len) { B->silu_mul(g, u, len); }
int or_b_logits(void* bp, size_t x, size_t y) {
    return guard([&] { B->logits(x, y); });
}
#undef B

}  // extern "C"

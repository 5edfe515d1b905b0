// TEST INFRASTRUCTURE ONLY: CPU restatement of the reference KernRT Q8 path.
// Compiled with -O2 -ffp-contract=off; see oracle.hpp for the rules.
#include "oracle.hpp"

#include <algorithm>
#include <cmath>
#include <random>
#include <cstring>
#include <stdexcept>

namespace oracle {

static inline uint32_t bits_of(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// Rust `f32::max`: IEEE maxNum, NaN-ignoring (same contract as fmaxf).
static inline float rmax(float a, float b) { return std::fmax(a, b); }

// Rust `(v * inv).round().clamp(-127.0, 127.0) as i8`: round half away from
// zero, clamp (NaN passes through), saturating cast (NaN -> 0).
static inline int8_t q8_round(float t) {
    float r = std::roundf(t);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    if (std::isnan(r)) return 0;
    return (int8_t)(int)r;
}

// quant.rs:722-758
uint16_t f32_to_f16_bits(float value) {
    uint32_t bits = bits_of(value);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exp = (int32_t)((bits >> 23) & 0xff) - 127 + 15;
    uint32_t mant = bits & 0x007fffff;
    if (((bits >> 23) & 0xff) == 0xff) {
        return (uint16_t)(sign | 0x7c00 | (mant != 0 ? 0x0200 : 0));
    }
    if (exp <= 0) {
        if (exp < -10) return sign;
        uint32_t significand = mant | 0x00800000;
        uint32_t shift = (uint32_t)(14 - exp);
        uint32_t base = significand >> shift;
        uint32_t rem = significand & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        uint32_t rounded = base + ((rem > halfway || (rem == halfway && (base & 1) != 0)) ? 1u : 0u);
        return (uint16_t)(sign | (uint16_t)rounded);
    }
    if (exp >= 31) return (uint16_t)(sign | 0x7c00);
    uint32_t base = mant >> 13;
    uint32_t rem = mant & 0x1fff;
    uint32_t rounded = base + ((rem > 0x1000 || (rem == 0x1000 && (base & 1) != 0)) ? 1u : 0u);
    int32_t e2 = exp;
    uint32_t m2 = rounded;
    if (rounded == 0x400) { e2 = exp + 1; m2 = 0; }
    if (e2 >= 31) return (uint16_t)(sign | 0x7c00);
    return (uint16_t)(sign | (uint16_t)((uint32_t)e2 << 10) | (uint16_t)m2);
}

// quant.rs:764-769
float f16_scale_to_f32(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits >> 15) << 31;
    uint32_t exp = (uint32_t)((bits >> 10) & 0x1f);
    uint32_t mant = (uint32_t)(bits & 0x03ff);
    return float_of(sign | ((exp + 112) << 23) | (mant << 13));
}

// dot.rs:222-224
float bf16_to_f32(uint16_t bits) { return float_of((uint32_t)bits << 16); }

// quant.rs:707-711
uint16_t f32_to_bf16_bits(float value) {
    uint32_t bits = bits_of(value);
    uint32_t lsb = (bits >> 16) & 1;
    return (uint16_t)((bits + 0x7fff + lsb) >> 16);
}

// quant.rs:856-874 (quantize, :831-851, has the same arithmetic)
void Q8Vec::quantize_into(const float* x, size_t n) {
    size_t blocks = (n + Q8_0_BLOCK - 1) / Q8_0_BLOCK;
    scales.clear();
    scales_f16.clear();
    quants.assign(blocks * Q8_0_BLOCK, 0);
    for (size_t b = 0; b < blocks; b++) {
        size_t lo = b * Q8_0_BLOCK, hi = std::min(n, lo + Q8_0_BLOCK);
        float amax = 0.0f;
        for (size_t i = lo; i < hi; i++) amax = rmax(amax, std::fabs(x[i]));
        float d = amax / 127.0f;
        float inv = d > 0.0f ? 1.0f / d : 0.0f;
        scales.push_back(d);
        scales_f16.push_back(f32_to_f16_bits(d));
        for (size_t i = lo; i < hi; i++) quants[i] = q8_round(x[i] * inv);
    }
}

Q8Vec Q8Vec::quantize(const float* x, size_t n) {
    Q8Vec q;
    q.quantize_into(x, n);
    return q;
}

Matrix Matrix::from_f32(std::vector<float> data, size_t out, size_t in) {
    Matrix m;
    m.kind = F32;
    m.out_dim = out;
    m.in_dim = in;
    m.f32 = std::move(data);
    return m;
}

Matrix Matrix::from_bf16_bits(std::vector<uint16_t> bits, size_t out, size_t in) {
    Matrix m;
    m.kind = BF16;
    m.out_dim = out;
    m.in_dim = in;
    m.bf16 = std::move(bits);
    return m;
}

// quant.rs:544-557
bool Matrix::from_f32_q8_0(const std::vector<float>& data, size_t out, size_t in, Matrix* m) {
    if (in % Q8_0_BLOCK != 0) return false;
    Q8Vec q = Q8Vec::quantize(data.data(), data.size());
    m->kind = Q8_0;
    m->out_dim = out;
    m->in_dim = in;
    m->scales = std::move(q.scales);
    m->quants = std::move(q.quants);
    return true;
}

// quant.rs:124-164
bool Matrix::from_f32_q8_0x4(const std::vector<float>& data, size_t out, size_t in, Matrix* m) {
    if (in % Q8_0_BLOCK != 0 || out % 4 != 0) return false;
    size_t groups = out / 4, blocks = in / Q8_0_BLOCK;
    m->kind = Q8_0X4;
    m->out_dim = out;
    m->in_dim = in;
    m->blocks.assign(groups * blocks, Q8Block4{});
    for (size_t g = 0; g < groups; g++) {
        for (size_t b = 0; b < blocks; b++) {
            Q8Block4& pb = m->blocks[g * blocks + b];
            std::memset(&pb, 0, sizeof pb);
            size_t col0 = b * Q8_0_BLOCK;
            for (size_t r = 0; r < 4; r++) {
                size_t row = g * 4 + r;
                const float* src = &data[row * in + col0];
                float amax = 0.0f;
                for (size_t i = 0; i < 32; i++) amax = rmax(amax, std::fabs(src[i]));
                float scale = amax / 127.0f;
                pb.scales[r] = f32_to_f16_bits(scale);
                float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
                for (size_t seg = 0; seg < 8; seg++)
                    for (size_t lane = 0; lane < 4; lane++)
                        pb.quants[seg * 16 + r * 4 + lane] = q8_round(src[seg * 4 + lane] * inv);
            }
        }
    }
    return true;
}

const char* Matrix::kind_name() const {
    switch (kind) {
        case F32: return "f32";
        case BF16: return "bf16";
        case Q8_0: return "q8_0";
        case Q8_0X4: return "q8_0x4";
    }
    return "?";
}

// quant.rs:659-693, quant.rs:174-190
void Matrix::decode_row(size_t index, float* out) const {
    size_t start = index * in_dim;
    switch (kind) {
        case F32:
            std::memcpy(out, &f32[start], in_dim * sizeof(float));
            break;
        case BF16:
            for (size_t i = 0; i < in_dim; i++) out[i] = bf16_to_f32(bf16[start + i]);
            break;
        case Q8_0: {
            size_t blocks = in_dim / Q8_0_BLOCK;
            for (size_t b = 0; b < blocks; b++) {
                float scale = scales[index * blocks + b];
                for (size_t i = 0; i < Q8_0_BLOCK; i++)
                    out[b * 32 + i] = (float)quants[start + b * 32 + i] * scale;
            }
            break;
        }
        case Q8_0X4: {
            size_t blocks = in_dim / Q8_0_BLOCK;
            size_t g = index / 4, r = index % 4;
            size_t o = 0;
            for (size_t b = 0; b < blocks; b++) {
                const Q8Block4& pb = blocks_at(g * blocks + b);
                float scale = f16_scale_to_f32(pb.scales[r]);
                for (size_t seg = 0; seg < 8; seg++)
                    for (size_t lane = 0; lane < 4; lane++)
                        out[o++] = (float)pb.quants[seg * 16 + r * 4 + lane] * scale;
            }
            break;
        }
    }
}

std::vector<float> Matrix::row(size_t index) const {
    std::vector<float> r(in_dim);
    decode_row(index, r.data());
    return r;
}

// quant.rs:597-612
std::vector<float> Matrix::to_f32_tensor() const {
    std::vector<float> all(out_dim * in_dim);
    for (size_t r = 0; r < out_dim; r++) decode_row(r, &all[r * in_dim]);
    return all;
}

// quant.rs:620-635
std::vector<uint16_t> Matrix::to_bf16_bits() const {
    if (kind == BF16) return bf16;
    std::vector<uint16_t> bits(out_dim * in_dim);
    if (kind == F32) {
        for (size_t i = 0; i < bits.size(); i++) bits[i] = f32_to_bf16_bits(f32[i]);
        return bits;
    }
    std::vector<float> row(in_dim);
    for (size_t r = 0; r < out_dim; r++) {
        decode_row(r, row.data());
        for (size_t i = 0; i < in_dim; i++) bits[r * in_dim + i] = f32_to_bf16_bits(row[i]);
    }
    return bits;
}

// quant.rs:198-219 (Q8_0x4) and quant.rs:646-652 (Q8_0 passthrough)
void Matrix::to_row_major(std::vector<int8_t>* q, std::vector<float>* s) const {
    if (kind == Q8_0) {
        *q = quants;
        *s = scales;
        return;
    }
    if (kind != Q8_0X4) throw std::runtime_error("to_row_major: not quantized");
    size_t blocks = in_dim / Q8_0_BLOCK;
    q->assign(out_dim * in_dim, 0);
    s->assign(out_dim * blocks, 0.0f);
    for (size_t g = 0; g < out_dim / Q8_0X4_ROWS; g++)
        for (size_t b = 0; b < blocks; b++) {
            const Q8Block4& pb = blocks_at(g * blocks + b);
            for (size_t r = 0; r < Q8_0X4_ROWS; r++) {
                size_t row = g * Q8_0X4_ROWS + r;
                (*s)[row * blocks + b] = f16_scale_to_f32(pb.scales[r]);
                int8_t* dst = &(*q)[row * in_dim + b * Q8_0_BLOCK];
                for (size_t seg = 0; seg < 8; seg++)
                    for (size_t lane = 0; lane < 4; lane++)
                        dst[seg * 4 + lane] = pb.quants[seg * 16 + r * 4 + lane];
            }
        }
}

// dot.rs:34-45
float dot_q8_0_scalar(const int8_t* a, const float* a_scales, const int8_t* b,
                      const float* b_scales, size_t blocks) {
    float total[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t blk = 0; blk < blocks; blk++) {
        size_t lo = blk * Q8_0_BLOCK;
        int32_t acc = 0;
        for (size_t i = 0; i < Q8_0_BLOCK; i++) acc += (int32_t)a[lo + i] * (int32_t)b[lo + i];
        float sa = a_scales[blk], sb = b_scales[blk];
        total[blk & 3] += (sa * sb) * (float)acc;
    }
    return ((total[0] + total[1]) + total[2]) + total[3];
}

// dot.rs:350-366
float dot_scalar(const float* a, const float* b, size_t n) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    size_t i = 0;
    while (i + 4 <= n) {
        acc[0] = std::fmaf(a[i], b[i], acc[0]);
        acc[1] = std::fmaf(a[i + 1], b[i + 1], acc[1]);
        acc[2] = std::fmaf(a[i + 2], b[i + 2], acc[2]);
        acc[3] = std::fmaf(a[i + 3], b[i + 3], acc[3]);
        i += 4;
    }
    float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    while (i < n) {
        sum = std::fmaf(a[i], b[i], sum);
        i++;
    }
    return sum;
}

// dot.rs:235-256
float dot_bf16_scalar(const uint16_t* a, const float* b, size_t n) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    size_t i = 0;
    while (i + 4 <= n) {
        for (int j = 0; j < 4; j++) acc[j] = std::fmaf(bf16_to_f32(a[i + j]), b[i + j], acc[j]);
        i += 4;
    }
    float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    while (i < n) {
        sum = std::fmaf(bf16_to_f32(a[i]), b[i], sum);
        i++;
    }
    return sum;
}

// reference.rs:73-79
float dot_plain(const float* a, const float* b, size_t n) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) sum += a[i] * b[i];
    return sum;
}

// quant.rs:223-236, the x86 branch: decode each row, re-quantize it, then
// run the row-wise Q8_0 dot with f32 activation scales.
void gemv_q8_0x4(const Matrix& w, const Q8Vec& qx, float* y) {
    for (size_t r = 0; r < w.out_dim; r++) {
        std::vector<float> row = w.row(r);
        Q8Vec row_q = Q8Vec::quantize(row.data(), row.size());
        size_t blocks = std::min(row_q.scales.size(), qx.scales.size());
        y[r] = dot_q8_0_scalar(row_q.quants.data(), row_q.scales.data(), qx.quants.data(),
                               qx.scales.data(), blocks);
    }
}

// quant.rs:23-62
void gemv_into(const Matrix& w, const float* x, float* y) {
    size_t in = w.in_dim, out = w.out_dim;
    switch (w.kind) {
        case Matrix::F32:
            for (size_t o = 0; o < out; o++) y[o] = dot_scalar(&w.f32[o * in], x, in);
            break;
        case Matrix::BF16:
            for (size_t o = 0; o < out; o++) y[o] = dot_bf16_scalar(&w.bf16[o * in], x, in);
            break;
        case Matrix::Q8_0: {
            Q8Vec qx = Q8Vec::quantize(x, in);
            size_t blocks = in / Q8_0_BLOCK;
            for (size_t o = 0; o < out; o++)
                y[o] = dot_q8_0_scalar(&w.quants[o * in], &w.scales[o * blocks], qx.quants.data(),
                                       qx.scales.data(), blocks);
            break;
        }
        case Matrix::Q8_0X4: {
            Q8Vec qx = Q8Vec::quantize(x, in);
            gemv_q8_0x4(w, qx, y);
            break;
        }
    }
}

// quant.rs:66-97
bool gemv_q8_0_into(const Matrix& w, const Q8Vec& qx, float* y) {
    size_t in = w.in_dim, out = w.out_dim;
    if (qx.quants.size() < in) return false;
    if (w.kind == Matrix::Q8_0) {
        size_t blocks = in / Q8_0_BLOCK;
        // `zip(a_scales, b_scales)` stops at the shorter of the two.
        size_t nb = std::min(blocks, qx.scales.size());
        for (size_t o = 0; o < out; o++)
            y[o] = dot_q8_0_scalar(&w.quants[o * in], &w.scales[o * blocks], qx.quants.data(),
                                   qx.scales.data(), nb);
        return true;
    }
    if (w.kind == Matrix::Q8_0X4) {
        gemv_q8_0x4(w, qx, y);
        return true;
    }
    return false;
}

// quant.rs:245-292 (portable loop :268-291)
void gemm_q8_0x4_batched_into(const Matrix& w, const int8_t* quants, const uint16_t* scales_f16,
                              size_t rows, float* y) {
    size_t in = w.in_dim, out = w.out_dim, blocks = in / Q8_0_BLOCK;
    for (size_t row = 0; row < rows; row++) {
        for (size_t g = 0; g < out / 4; g++) {
            float* o = &y[row * out + g * 4];
            for (int i = 0; i < 4; i++) o[i] = 0.0f;
            for (size_t b = 0; b < blocks; b++) {
                const Q8Block4& pb = w.blocks_at(g * blocks + b);
                float xs = f16_scale_to_f32(scales_f16[row * blocks + b]);
                for (size_t lane = 0; lane < 4; lane++) {
                    float ws = f16_scale_to_f32(pb.scales[lane]) * xs;
                    int32_t sum = 0;
                    for (size_t seg = 0; seg < 8; seg++)
                        for (size_t byte = 0; byte < 4; byte++)
                            sum += (int32_t)pb.quants[seg * 16 + lane * 4 + byte] *
                                   (int32_t)quants[row * in + b * 32 + seg * 4 + byte];
                    o[lane] = std::fmaf((float)sum, ws, o[lane]);
                }
            }
        }
    }
}

// elementwise.rs:81-91
void softmax_in_place(float* x, size_t n) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = rmax(mx, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = std::exp(x[i] - mx);
        sum += x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

// generate.rs:70-77
size_t argmax(const float* v, size_t n) {
    auto key = [](float f) {
        int32_t k = (int32_t)bits_of(f);
        k ^= (int32_t)(((uint32_t)(k >> 31)) >> 1);
        return k;
    };
    size_t best = 0;
    int32_t best_key = key(v[0]);
    for (size_t i = 1; i < n; i++) {
        int32_t k = key(v[i]);
        if (k >= best_key) {  // max_by keeps the last of equal maxima
            best_key = k;
            best = i;
        }
    }
    return best;
}

// tests/backends.rs:41-51
std::vector<float> lcg_fill(size_t count, uint64_t seed) {
    std::vector<float> out(count);
    uint64_t state = seed;
    for (size_t i = 0; i < count; i++) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        out[i] = ((float)(state >> 40) / (float)(1ULL << 24)) - 0.5f;
    }
    return out;
}

// mod.rs:72-84
const Matrix* LayerWeights::matrix_opt(Proj p) const {
    switch (p) {
        case Proj::Q: return wq.get();
        case Proj::K: return wk.get();
        case Proj::V: return wv.get();
        case Proj::O: return wo.get();
        case Proj::Gate: return &w1;
        case Proj::Down: return &w2;
        case Proj::Up: return &w3;
        case Proj::ConvIn: return conv_in.get();
        case Proj::ConvOut: return conv_out.get();
    }
    return nullptr;
}

// ---------------------------------------------------------------------------
// Shared scalar helpers of cpu.rs / reference.rs

static float silu(float x) { return x / (1.0f + std::exp(-x)); }  // cpu.rs:708-710

// cpu.rs:557-571 / reference.rs:490-503
static void conv_rows(const float* x, const float* kernel, float* out, size_t rows, size_t dim,
                      size_t k) {
    for (size_t r = 0; r < rows; r++)
        for (size_t i = 0; i < dim; i++) {
            float acc = 0.0f;
            for (size_t j = 0; j < k; j++) {
                long h = (long)r - ((long)k - 1) + (long)j;
                if (h >= 0) acc += kernel[i * k + j] * x[(size_t)h * dim + i];
            }
            out[r * dim + i] = acc;
        }
}

// cpu.rs:633-644
static void rms_norm_row(float* out, const float* x, const float* w, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    ss /= (float)n;
    ss += eps;
    float scale = 1.0f / std::sqrt(ss);
    for (size_t i = 0; i < n; i++) out[i] = w[i] * (scale * x[i]);
}

// cpu.rs:664-690
static void rope_interleaved(float* q, size_t qlen, float* k, size_t pos, size_t head_size,
                             size_t kv_dim, float theta) {
    size_t i = 0;
    while (i + 1 < qlen) {
        size_t head_dim = i % head_size;
        float freq = 1.0f / std::pow(theta, (float)head_dim / (float)head_size);
        float angle = (float)pos * freq;
        float s = std::sin(angle), c = std::cos(angle);
        float q0 = q[i], q1 = q[i + 1];
        q[i] = q0 * c - q1 * s;
        q[i + 1] = q0 * s + q1 * c;
        if (i < kv_dim) {
            float k0 = k[i], k1 = k[i + 1];
            k[i] = k0 * c - k1 * s;
            k[i + 1] = k0 * s + k1 * c;
        }
        i += 2;
    }
}

// cpu.rs:693-705
static void rope_half(float* v, size_t len, size_t pos, size_t head_size, float theta) {
    size_t half = head_size / 2;
    for (size_t h = 0; h + head_size <= len; h += head_size) {
        float* head = v + h;
        for (size_t i = 0; i < half; i++) {
            float freq = 1.0f / std::pow(theta, (float)(2 * i) / (float)head_size);
            float angle = (float)pos * freq;
            float s = std::sin(angle), c = std::cos(angle);
            float lo = head[i], hi = head[i + half];
            head[i] = lo * c - hi * s;
            head[i + half] = lo * s + hi * c;
        }
    }
}

// The buffer table, KV cache and the ops both scalar backends share verbatim
// (copy, kv_write, add, mul, conv, silu_mul); rms_norm, qk_norm and rope here
// follow cpu.rs, and the Reference backend below overrides them with its own
// transcription of reference.rs.
class HostBackend : public Backend {
protected:
    std::shared_ptr<const ModelWeights> w_;
    const char* storage_ = "f32";
    std::vector<std::vector<float>> bufs_;
    std::vector<float> kc_, vc_;
    KvSpec kv_{0, 0, 0};
    const ModelWeights& weights() const {
        if (!w_) throw std::runtime_error("prepare() runs before any compute");
        return *w_;
    }

public:
    const char* storage() const override { return storage_; }
    void prepare(std::shared_ptr<const ModelWeights> w, KvSpec kv) override {
        storage_ = w->token_embedding.kind_name();
        kv_ = kv;
        kc_.assign(kv.n_layers * kv.seq_len * kv.kv_dim, 0.0f);
        vc_.assign(kv.n_layers * kv.seq_len * kv.kv_dim, 0.0f);
        w_ = std::move(w);
    }
    Buf alloc(size_t len) override {
        bufs_.emplace_back(len, 0.0f);
        return bufs_.size() - 1;
    }
    Buf upload(const float* data, size_t len) override {
        bufs_.emplace_back(data, data + len);
        return bufs_.size() - 1;
    }
    void read(Buf src, float* out, size_t len) override {
        std::memcpy(out, bufs_.at(src).data(), len * sizeof(float));
    }
    void embed(size_t token, Buf out, size_t offset) override {
        weights().token_embedding.decode_row(token, &bufs_.at(out)[offset]);
    }
    // cpu.rs:229-236: memmove when src == dst
    void copy(Buf src, size_t so, Buf dst, size_t doff, size_t len) override {
        std::memmove(&bufs_.at(dst)[doff], &bufs_.at(src)[so], len * sizeof(float));
    }
    // cpu.rs:238-246
    void kv_write(size_t layer, const size_t* slots, Buf k, Buf v, size_t rows) override {
        size_t width = kv_.kv_dim;
        for (size_t row = 0; row < rows; row++) {
            size_t at = (layer * kv_.seq_len + slots[row]) * width;
            std::memcpy(&kc_[at], &bufs_.at(k)[row * width], width * sizeof(float));
            std::memcpy(&vc_[at], &bufs_.at(v)[row * width], width * sizeof(float));
        }
    }
    // cpu.rs:248-255 + rms_norm_row cpu.rs:633-644
    void rms_norm(Buf out, Buf x, Buf w, size_t rows, size_t dim, float eps) override {
        std::vector<float> wv = bufs_.at(w);
        for (size_t r = 0; r < rows; r++)
            rms_norm_row(&bufs_.at(out)[r * dim], &bufs_.at(x)[r * dim], wv.data(), dim, eps);
    }
    // cpu.rs:257-272 + qk_norm_row cpu.rs:647-661
    void qk_norm(Buf v, size_t rows, size_t width, size_t head, Buf w, float eps) override {
        std::vector<float> wv = bufs_.at(w);
        float* data = bufs_.at(v).data();
        for (size_t r = 0; r < rows; r++)
            for (size_t h = 0; h + head <= width; h += head) {
                float* hd = data + r * width + h;
                rms_norm_row(hd, hd, wv.data(), head, eps);
            }
    }
    // cpu.rs:274-302 + rope_interleaved / rope_half cpu.rs:664-705
    void rope(Buf q, Buf k, size_t qw, size_t kvw, size_t rows, const size_t* positions,
              RopeSpec spec) override {
        for (size_t r = 0; r < rows; r++) {
            float* qv = &bufs_.at(q)[r * qw];
            float* kv = &bufs_.at(k)[r * kvw];
            if (spec.interleaved) {
                rope_interleaved(qv, qw, kv, positions[r], spec.head_size, kvw, spec.theta);
            } else {
                rope_half(qv, qw, positions[r], spec.head_size, spec.theta);
                rope_half(kv, kvw, positions[r], spec.head_size, spec.theta);
            }
        }
    }
    void add_in_place(Buf dst, Buf src, size_t len) override {
        float* d = bufs_.at(dst).data();
        const float* s = bufs_.at(src).data();
        for (size_t i = 0; i < len; i++) d[i] += s[i];
    }
    // cpu.rs:412-460: element by element, reads before the write
    void mul(Buf out, size_t oo, Buf a, size_t ao, Buf b, size_t bo, size_t len) override {
        for (size_t i = 0; i < len; i++) {
            float x = bufs_.at(a)[ao + i];
            float y = bufs_.at(b)[bo + i];
            bufs_.at(out)[oo + i] = x * y;
        }
    }
    void conv_prefill(Buf out, Buf x, Buf kernel, size_t rows, size_t dim, size_t k) override {
        std::vector<float> xv = bufs_.at(x), kv = bufs_.at(kernel);
        conv_rows(xv.data(), kv.data(), bufs_.at(out).data(), rows, dim, k);
    }
    // cpu.rs:469-492
    void conv_decode(Buf out, Buf x, Buf kernel, Buf state, size_t dim, size_t k) override {
        std::vector<float> sv = bufs_.at(state), xv = bufs_.at(x), kv = bufs_.at(kernel);
        size_t hist_len = k - 1;
        std::vector<float> hist(sv.begin(), sv.begin() + hist_len * dim);
        hist.insert(hist.end(), xv.begin(), xv.begin() + dim);
        std::vector<float> full(k * dim, 0.0f);
        conv_rows(hist.data(), kv.data(), full.data(), k, dim, k);
        std::memcpy(bufs_.at(out).data(), &full[(k - 1) * dim], dim * sizeof(float));
        if (hist_len > 0) {
            float* s = bufs_.at(state).data();
            if (hist_len > 1) std::memmove(s, s + dim, (hist_len - 1) * dim * sizeof(float));
            std::memcpy(s + (hist_len - 1) * dim, xv.data(), dim * sizeof(float));
        }
    }
    void fill_kv(size_t slots, uint64_t seed) {
        std::mt19937_64 rng(seed);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        for (size_t l = 0; l < kv_.n_layers; l++)
            for (size_t i = 0; i < slots * kv_.kv_dim; i++) {
                size_t at = l * kv_.seq_len * kv_.kv_dim + i;
                kc_[at] = nd(rng);
                vc_[at] = nd(rng);
            }
    }
    // test set-up: data into the key (which 0) or value (1) cache at an
    // element offset of [n_layers, seq_len, kv_dim]
    void set_kv(int which, size_t offset, const float* data, size_t len) {
        std::vector<float>& c = which == 0 ? kc_ : vc_;
        if (offset + len > c.size()) throw std::runtime_error("kv upload past the cache");
        std::memcpy(&c[offset], data, len * sizeof(float));
    }
    void silu_mul(Buf gate, Buf up, size_t len) override {
        float* g = bufs_.at(gate).data();
        const float* u = bufs_.at(up).data();
        for (size_t i = 0; i < len; i++) g[i] = silu(g[i]) * u[i];
    }
};

// cpu.rs:31-515 with prefill_f32 = false
class Cpu : public HostBackend {
    Q8Vec q8_;
    std::vector<int8_t> batch_quants_;
    std::vector<uint16_t> batch_scales_f16_;

    // cpu.rs:143-158
    void quantize_rows(const float* input, size_t width, size_t rows) {
        size_t blocks = width / Q8_0_BLOCK;
        batch_quants_.assign(rows * width, 0);
        batch_scales_f16_.assign(rows * blocks, 0);
        for (size_t r = 0; r < rows; r++) {
            q8_.quantize_into(input + r * width, width);
            std::memcpy(&batch_quants_[r * width], q8_.quants.data(), width);
            std::memcpy(&batch_scales_f16_[r * blocks], q8_.scales_f16.data(), blocks * 2);
        }
    }

public:
    const char* name() const override { return "cpu"; }

    // cpu.rs:304-371 (prefill_f32 == false branches)
    void project(size_t layer, Proj p, Buf x, Buf y, size_t rows) override {
        const Matrix* w = weights().layers.at(layer).matrix_opt(p);
        if (!w) throw std::runtime_error("projection is not live on this layer");
        size_t in = w->in_dim, out = w->out_dim;
        if (w->kind == Matrix::Q8_0X4) {
            std::vector<float> xv = bufs_.at(x);
            quantize_rows(xv.data(), in, rows);
            gemm_q8_0x4_batched_into(*w, batch_quants_.data(), batch_scales_f16_.data(), rows,
                                     bufs_.at(y).data());
            return;
        }
        bool quantized = w->kind == Matrix::Q8_0;
        for (size_t r = 0; r < rows; r++) {
            const float* src = &bufs_.at(x)[r * in];
            float* dst = &bufs_.at(y)[r * out];
            if (quantized) {
                q8_.quantize_into(src, in);
                if (!gemv_q8_0_into(*w, q8_, dst)) throw std::runtime_error("shapes are fixed at load");
            } else {
                gemv_into(*w, src, dst);
            }
        }
    }

    // cpu.rs:373-403 + attention_rows cpu.rs:575-630
    void attention(Buf q, Buf out, Buf att, size_t layer, const Window* windows, size_t n_windows,
                   AttnSpec spec) override {
        std::vector<float> qv = bufs_.at(q);
        size_t loff = layer * spec.seq_len * spec.kv_dim;
        size_t width = spec.n_heads * spec.head_size;
        float scale = 1.0f / std::sqrt((float)spec.head_size);
        for (size_t row = 0; row < n_windows; row++) {
            const Window& w = windows[row];
            size_t n_shared = w.shared_end - w.shared_start;
            size_t count = n_shared + w.slot - w.att_start + 1;
            for (size_t h = 0; h < spec.n_heads; h++) {
                const float* qh = &qv[row * width + h * spec.head_size];
                float* sc = &bufs_.at(att)[row * spec.n_heads * spec.seq_len + h * spec.seq_len];
                size_t kvo = (h / spec.kv_mul) * spec.head_size;
                size_t i = 0;
                for (size_t t = w.shared_start; t < w.shared_end; t++, i++)
                    sc[i] = dot_scalar(qh, &kc_[loff + t * spec.kv_dim + kvo], spec.head_size) * scale;
                for (size_t t = w.att_start; t <= w.slot; t++, i++)
                    sc[i] = dot_scalar(qh, &kc_[loff + t * spec.kv_dim + kvo], spec.head_size) * scale;
                softmax_in_place(sc, count);
                float* o = &bufs_.at(out)[row * width + h * spec.head_size];
                for (size_t e = 0; e < spec.head_size; e++) o[e] = 0.0f;
                i = 0;
                for (size_t t = w.shared_start; t < w.shared_end; t++, i++) {
                    float a = sc[i];
                    const float* vv = &vc_[loff + t * spec.kv_dim + kvo];
                    for (size_t e = 0; e < spec.head_size; e++) o[e] += a * vv[e];
                }
                for (size_t t = w.att_start; t <= w.slot; t++, i++) {
                    float a = sc[i];
                    const float* vv = &vc_[loff + t * spec.kv_dim + kvo];
                    for (size_t e = 0; e < spec.head_size; e++) o[e] += a * vv[e];
                }
            }
        }
    }

    // cpu.rs:501-514
    void logits(Buf x, Buf y) override {
        const Matrix& w = weights().classifier();
        const std::vector<float>& xv = bufs_.at(x);
        if (w.kind == Matrix::Q8_0 || w.kind == Matrix::Q8_0X4) {
            q8_.quantize_into(xv.data(), xv.size());
            if (!gemv_q8_0_into(w, q8_, bufs_.at(y).data()))
                throw std::runtime_error("shapes are fixed at load");
        } else {
            gemv_into(w, xv.data(), bufs_.at(y).data());
        }
    }
};

// reference.rs:44-485
class Reference : public HostBackend {
public:
    const char* name() const override { return "reference"; }

    // reference.rs:160-176, transcribed on its own (index arithmetic over the
    // flat buffers) rather than through the cpu backend's rms_norm_row, so
    // that cpu-vs-reference agreement checks one transcription against the other.
    void rms_norm(Buf out, Buf x, Buf weight, size_t rows, size_t dim, float eps) override {
        std::vector<float> w = bufs_.at(weight);
        std::vector<float>& xi = bufs_.at(x);
        for (size_t row = 0; row < rows; row++) {
            size_t at = row * dim;
            float ss = 0.0f;
            for (size_t i = 0; i < dim; i++) ss += xi[at + i] * xi[at + i];
            ss /= (float)dim;
            ss += eps;
            float scale = 1.0f / std::sqrt(ss);
            std::vector<float>& o = bufs_.at(out);
            for (size_t i = 0; i < dim; i++) o[at + i] = w[i] * (scale * xi[at + i]);
        }
    }

    // reference.rs:178-207
    void qk_norm(Buf v, size_t rows, size_t width, size_t head_size, Buf weight, float eps) override {
        std::vector<float> w = bufs_.at(weight);
        std::vector<float>& data = bufs_.at(v);
        for (size_t row = 0; row < rows; row++) {
            size_t base = row * width;
            for (size_t head = 0; head < width / head_size; head++) {
                size_t at = base + head * head_size;
                float ss = 0.0f;
                for (size_t i = 0; i < head_size; i++) ss += data[at + i] * data[at + i];
                ss /= (float)head_size;
                ss += eps;
                float scale = 1.0f / std::sqrt(ss);
                for (size_t i = 0; i < head_size; i++) data[at + i] = w[i] * (scale * data[at + i]);
            }
        }
    }

    // reference.rs:209-257
    void rope(Buf q, Buf k, size_t q_width, size_t kv_width, size_t rows, const size_t* positions,
              RopeSpec spec) override {
        std::vector<float>& qv = bufs_.at(q);
        std::vector<float>& kv = bufs_.at(k);
        for (size_t row = 0; row < rows; row++) {
            size_t pos = positions[row];
            size_t qo = row * q_width, ko = row * kv_width;
            if (spec.interleaved) {
                for (size_t i = 0; i + 1 < q_width; i += 2) {
                    size_t head_dim = i % spec.head_size;
                    float freq = 1.0f / std::pow(spec.theta, (float)head_dim / (float)spec.head_size);
                    float angle = (float)pos * freq;
                    float sn = std::sin(angle), cs = std::cos(angle);
                    float q0 = qv[qo + i], q1 = qv[qo + i + 1];
                    qv[qo + i] = q0 * cs - q1 * sn;
                    qv[qo + i + 1] = q0 * sn + q1 * cs;
                    if (i < kv_width) {
                        float k0 = kv[ko + i], k1 = kv[ko + i + 1];
                        kv[ko + i] = k0 * cs - k1 * sn;
                        kv[ko + i + 1] = k0 * sn + k1 * cs;
                    }
                }
            } else {
                size_t half = spec.head_size / 2;
                std::vector<float>* vecs[2] = {&qv, &kv};
                size_t bases[2] = {qo, ko}, widths[2] = {q_width, kv_width};
                for (int s = 0; s < 2; s++) {
                    std::vector<float>& vec = *vecs[s];
                    for (size_t head = 0; head < widths[s] / spec.head_size; head++) {
                        size_t at = bases[s] + head * spec.head_size;
                        for (size_t i = 0; i < half; i++) {
                            float freq = 1.0f / std::pow(spec.theta, (float)(2 * i) / (float)spec.head_size);
                            float angle = (float)pos * freq;
                            float sn = std::sin(angle), cs = std::cos(angle);
                            float lo = vec[at + i], hi = vec[at + i + half];
                            vec[at + i] = lo * cs - hi * sn;
                            vec[at + i + half] = lo * sn + hi * cs;
                        }
                    }
                }
            }
        }
    }

    // reference.rs:259-274
    void project(size_t layer, Proj p, Buf x, Buf y, size_t rows) override {
        const Matrix* w = weights().layers.at(layer).matrix_opt(p);
        if (!w) throw std::runtime_error("projection is not live on this layer");
        size_t in = w->in_dim, out = w->out_dim;
        std::vector<float> row(in);
        for (size_t r = 0; r < rows; r++) {
            const float* src = &bufs_.at(x)[r * in];
            float* dst = &bufs_.at(y)[r * out];
            for (size_t o = 0; o < out; o++) {
                w->decode_row(o, row.data());
                dst[o] = dot_plain(row.data(), src, in);
            }
        }
    }

    // reference.rs:276-306 + attention_rows reference.rs:418-484
    void attention(Buf q, Buf out, Buf att, size_t layer, const Window* windows, size_t n_windows,
                   AttnSpec spec) override {
        std::vector<float> qv = bufs_.at(q);
        size_t loff = layer * spec.seq_len * spec.kv_dim;
        size_t width = spec.n_heads * spec.head_size;
        float scale = 1.0f / std::sqrt((float)spec.head_size);
        for (size_t row = 0; row < n_windows; row++) {
            const Window& w = windows[row];
            size_t n_shared = w.shared_end - w.shared_start;
            size_t count = n_shared + w.slot - w.att_start + 1;
            for (size_t h = 0; h < spec.n_heads; h++) {
                const float* qh = &qv[row * width + h * spec.head_size];
                float* sc = &bufs_.at(att)[row * spec.n_heads * spec.seq_len + h * spec.seq_len];
                size_t kvo = (h / spec.kv_mul) * spec.head_size;
                size_t i = 0;
                for (size_t t = w.shared_start; t < w.shared_end; t++, i++)
                    sc[i] = dot_plain(qh, &kc_[loff + t * spec.kv_dim + kvo], spec.head_size) * scale;
                for (size_t t = w.att_start; t <= w.slot; t++, i++)
                    sc[i] = dot_plain(qh, &kc_[loff + t * spec.kv_dim + kvo], spec.head_size) * scale;
                float mx = -INFINITY;
                for (size_t j = 0; j < count; j++)
                    if (sc[j] > mx) mx = sc[j];
                float sum = 0.0f;
                for (size_t j = 0; j < count; j++) {
                    sc[j] = std::exp(sc[j] - mx);
                    sum += sc[j];
                }
                for (size_t j = 0; j < count; j++) sc[j] /= sum;
                float* o = &bufs_.at(out)[row * width + h * spec.head_size];
                for (size_t e = 0; e < spec.head_size; e++) o[e] = 0.0f;
                i = 0;
                for (size_t t = w.shared_start; t < w.shared_end; t++, i++) {
                    float a = sc[i];
                    for (size_t e = 0; e < spec.head_size; e++) o[e] += a * vc_[loff + t * spec.kv_dim + kvo + e];
                }
                for (size_t t = w.att_start; t <= w.slot; t++, i++) {
                    float a = sc[i];
                    for (size_t e = 0; e < spec.head_size; e++) o[e] += a * vc_[loff + t * spec.kv_dim + kvo + e];
                }
            }
        }
    }

    // reference.rs:402-414
    void logits(Buf x, Buf y) override {
        const Matrix& w = weights().classifier();
        std::vector<float> row(w.in_dim);
        const float* src = bufs_.at(x).data();
        for (size_t o = 0; o < w.out_dim; o++) {
            w.decode_row(o, row.data());
            bufs_.at(y)[o] = dot_plain(row.data(), src, w.in_dim);
        }
    }
};

std::unique_ptr<Backend> make_cpu() { return std::unique_ptr<Backend>(new Cpu()); }
void fill_kv(Backend& b, size_t slots, uint64_t seed) { dynamic_cast<HostBackend&>(b).fill_kv(slots, seed); }
void set_kv(Backend& b, int which, size_t offset, const float* data, size_t len) {
    dynamic_cast<HostBackend&>(b).set_kv(which, offset, data, len);
}
std::unique_ptr<Backend> make_reference() { return std::unique_ptr<Backend>(new Reference()); }

// ---------------------------------------------------------------------------
// Llama driver, arch/llm/llama.rs

Llama::Llama(Config c, std::shared_ptr<const ModelWeights> w, std::unique_ptr<Backend> b)
    : c_(c), w_(std::move(w)), backend_(std::move(b)) {
    backend_->prepare(w_, KvSpec{c_.n_layers, c_.kv_dim(), c_.seq_len});  // :364-375
    for (const LayerWeights& l : w_->layers) {                              // :376-385
        Norms n{};
        n.att = backend_->upload(l.rms_att.data(), l.rms_att.size());
        n.ffn = backend_->upload(l.rms_ffn.data(), l.rms_ffn.size());
        n.has_q = !l.rms_q.empty();
        n.has_k = !l.rms_k.empty();
        if (n.has_q) n.q = backend_->upload(l.rms_q.data(), l.rms_q.size());
        if (n.has_k) n.k = backend_->upload(l.rms_k.data(), l.rms_k.size());
        norms_.push_back(n);
    }
    rms_final_ = backend_->upload(w_->rms_final.data(), w_->rms_final.size());
    size_t dim = c_.dim, kv = c_.kv_dim(), qd = c_.q_dim();                 // :387-407
    x_ = backend_->alloc(dim);
    xb_ = backend_->alloc(dim);
    q_ = backend_->alloc(qd);
    k_ = backend_->alloc(kv);
    v_ = backend_->alloc(kv);
    attn_ = backend_->alloc(qd);
    o_ = backend_->alloc(dim);
    gate_ = backend_->alloc(c_.hidden_dim);
    up_ = backend_->alloc(c_.hidden_dim);
    mlp_ = backend_->alloc(dim);
    hidden_ = backend_->alloc(dim);
    att_ = backend_->alloc(c_.n_heads * c_.seq_len);
    logits_ = backend_->alloc(c_.vocab_size);
    logits_host_.assign(c_.vocab_size, 0.0f);
}

// llama.rs:786-862
const std::vector<float>& Llama::forward(size_t token, size_t pos) {
    size_t dim = c_.dim, hidden = c_.hidden_dim, qd = c_.q_dim(), kv = c_.kv_dim();
    size_t hs = c_.head_dim;
    float eps = c_.rms_eps;
    AttnSpec as{c_.n_heads, c_.kv_mul(), hs, kv, c_.seq_len};
    RopeSpec rs{hs, c_.rope_theta, c_.rope_interleaved};
    size_t positions[1] = {pos};
    Backend& b = *backend_;
    b.embed(token, x_, 0);
    for (size_t l = 0; l < c_.n_layers; l++) {
        const Norms& n = norms_[l];
        b.rms_norm(xb_, x_, n.att, 1, dim, eps);
        b.project_qkv(l, xb_, q_, k_, v_, 1);
        if (n.has_q) b.qk_norm(q_, 1, qd, hs, n.q, eps);
        if (n.has_k) b.qk_norm(k_, 1, kv, hs, n.k, eps);
        b.rope(q_, k_, qd, kv, 1, positions, rs);
        b.kv_write(l, positions, k_, v_, 1);
        Window win{0, pos, 0, 0};
        b.attention(q_, attn_, att_, l, &win, 1, as);
        b.project(l, Proj::O, attn_, o_, 1);
        b.add_in_place(x_, o_, dim);
        b.rms_norm(xb_, x_, n.ffn, 1, dim, eps);
        b.project_gate_up(l, xb_, gate_, up_, 1);
        b.silu_mul(gate_, up_, hidden);
        b.project(l, Proj::Down, gate_, mlp_, 1);
        b.add_in_place(x_, mlp_, dim);
    }
    b.rms_norm(xb_, x_, rms_final_, 1, dim, eps);
    b.logits(xb_, logits_);
    b.read(logits_, logits_host_.data(), logits_host_.size());
    return logits_host_;
}

// llama.rs:473-492
const std::vector<float>& Llama::prefill(const size_t* tokens, size_t n, size_t start) {
    if (start + n > c_.seq_len) throw std::runtime_error("prefill runs past the context length");
    if (n == 0) return logits_host_;
    std::string st = storage();
    if (st != "f32" && st != "bf16" && st != "q8_0x4") {
        for (size_t i = 0; i < n; i++) forward(tokens[i], start + i);
        return logits_host_;
    }
    prefill_batched(tokens, n, start);
    return logits_host_;
}

// llama.rs:501-536
void Llama::prefill_batched(const size_t* tokens, size_t n, size_t start) {
    std::vector<PrefillRow> rows;
    for (size_t i = 0; i < n; i++) rows.push_back({tokens[i], start + i, start + i, 0, 0, 0});
    prefill_rows(rows);
    size_t dim = c_.dim;
    backend_->copy(pb_.x, (n - 1) * dim, hidden_, 0, dim);
    backend_->rms_norm(xb_, hidden_, rms_final_, 1, dim, c_.rms_eps);
    backend_->logits(xb_, logits_);
    backend_->read(logits_, logits_host_.data(), logits_host_.size());
}

// llama.rs:552-580
std::vector<std::vector<float>> Llama::prefill_multi(const std::vector<std::vector<size_t>>& seqs) {
    std::vector<PrefillRow> rows;
    std::vector<long> last_rows;
    size_t offset = 0;
    for (const auto& seq : seqs) {
        if (seq.empty()) { last_rows.push_back(-1); continue; }
        if (offset + seq.size() > c_.seq_len) throw std::runtime_error("prefill_multi runs past the context length");
        for (size_t i = 0; i < seq.size(); i++) rows.push_back({seq[i], i, offset + i, offset, 0, 0});
        last_rows.push_back((long)rows.size() - 1);
        offset += seq.size();
    }
    prefill_rows(rows);
    return final_hiddens(last_rows);
}

// llama.rs:603-647
std::vector<std::vector<float>> Llama::prefill_shared(const std::vector<size_t>& prefix,
                                                      const std::vector<std::vector<size_t>>& suffixes) {
    if (prefix.size() > c_.seq_len) throw std::runtime_error("prefill_shared prefix runs past the context length");
    std::vector<PrefillRow> rows;
    for (size_t i = 0; i < prefix.size(); i++) rows.push_back({prefix[i], i, i, 0, 0, 0});
    std::vector<long> last_rows;
    size_t base = prefix.size();
    for (const auto& suf : suffixes) {
        if (suf.empty()) { last_rows.push_back(-1); continue; }
        if (base + suf.size() > c_.seq_len) throw std::runtime_error("prefill_shared runs past the context length");
        for (size_t i = 0; i < suf.size(); i++)
            rows.push_back({suf[i], prefix.size() + i, base + i, base, 0, prefix.size()});
        last_rows.push_back((long)rows.size() - 1);
        base += suf.size();
    }
    prefill_rows(rows);
    return final_hiddens(last_rows);
}

// llama.rs:652-683
std::vector<std::vector<float>> Llama::final_hiddens(const std::vector<long>& rows) {
    std::vector<std::vector<float>> out;
    size_t dim = c_.dim;
    for (long r : rows) {
        if (r < 0) { out.emplace_back(dim, 0.0f); continue; }
        backend_->copy(pb_.x, (size_t)r * dim, hidden_, 0, dim);
        backend_->rms_norm(xb_, hidden_, rms_final_, 1, dim, c_.rms_eps);
        std::vector<float> h(dim);
        backend_->read(xb_, h.data(), dim);
        out.push_back(std::move(h));
    }
    return out;
}

// llama.rs:690-771
void Llama::prefill_rows(const std::vector<PrefillRow>& rows) {
    size_t n_tok = rows.size();
    size_t dim = c_.dim, hidden = c_.hidden_dim, qd = c_.q_dim(), kv = c_.kv_dim();
    size_t hs = c_.head_dim;
    float eps = c_.rms_eps;
    AttnSpec as{c_.n_heads, c_.kv_mul(), hs, kv, c_.seq_len};
    RopeSpec rs{hs, c_.rope_theta, c_.rope_interleaved};
    std::vector<size_t> positions, slots;
    std::vector<Window> windows;
    for (const PrefillRow& r : rows) {
        positions.push_back(r.rope_pos);
        slots.push_back(r.slot);
        windows.push_back({r.att_start, r.slot, r.sh_start, r.sh_end});
    }
    Backend& b = *backend_;
    if (!has_prefill_ || pb_.n_tok < n_tok) {  // :729-731, PrefillBuffers::new :148-166
        pb_ = PrefillBuffers{n_tok,
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * qd),
                             b.alloc(n_tok * kv),
                             b.alloc(n_tok * kv),
                             b.alloc(n_tok * qd),
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * hidden),
                             b.alloc(n_tok * hidden),
                             b.alloc(n_tok * c_.n_heads * c_.seq_len)};
        has_prefill_ = true;
    }
    for (size_t r = 0; r < n_tok; r++) b.embed(rows[r].token, pb_.x, r * dim);
    for (size_t l = 0; l < c_.n_layers; l++) {
        const Norms& n = norms_[l];
        b.rms_norm(pb_.xb, pb_.x, n.att, n_tok, dim, eps);
        b.project_qkv(l, pb_.xb, pb_.q, pb_.k, pb_.v, n_tok);
        if (n.has_q) b.qk_norm(pb_.q, n_tok, qd, hs, n.q, eps);
        if (n.has_k) b.qk_norm(pb_.k, n_tok, kv, hs, n.k, eps);
        b.rope(pb_.q, pb_.k, qd, kv, n_tok, positions.data(), rs);
        b.kv_write(l, slots.data(), pb_.k, pb_.v, n_tok);
        b.attention(pb_.q, pb_.attn, pb_.att, l, windows.data(), windows.size(), as);
        b.project(l, Proj::O, pb_.attn, pb_.o, n_tok);
        b.add_in_place(pb_.x, pb_.o, n_tok * dim);
        b.rms_norm(pb_.xb, pb_.x, n.ffn, n_tok, dim, eps);
        b.project_gate_up(l, pb_.xb, pb_.gate, pb_.up, n_tok);
        b.silu_mul(pb_.gate, pb_.up, n_tok * hidden);
        b.project(l, Proj::Down, pb_.gate, pb_.o, n_tok);
        b.add_in_place(pb_.x, pb_.o, n_tok * dim);
    }
}

// ---------------------------------------------------------------------------
// LFM2 driver, arch/llm/lfm2.rs

Lfm2::Lfm2(Config c, std::vector<bool> is_attention, std::shared_ptr<const ModelWeights> w,
           std::unique_ptr<Backend> b)
    : c_(c), is_attention_(std::move(is_attention)), w_(std::move(w)), backend_(std::move(b)) {
    if (is_attention_.size() != c_.n_layers) throw std::runtime_error("layer mask must cover every layer");
    backend_->prepare(w_, KvSpec{c_.n_layers, c_.kv_dim(), c_.seq_len});  // :284-291
    for (const LayerWeights& l : w_->layers) {                              // :293-301
        Norms n{};
        n.op = backend_->upload(l.rms_att.data(), l.rms_att.size());
        n.ffn = backend_->upload(l.rms_ffn.data(), l.rms_ffn.size());
        n.has_q = !l.rms_q.empty();
        n.has_k = !l.rms_k.empty();
        if (n.has_q) n.q = backend_->upload(l.rms_q.data(), l.rms_q.size());
        if (n.has_k) n.k = backend_->upload(l.rms_k.data(), l.rms_k.size());
        norms_.push_back(n);
    }
    rms_final_ = backend_->upload(w_->rms_final.data(), w_->rms_final.size());
    size_t dim = c_.dim;
    for (const LayerWeights& l : w_->layers) {  // :306-330
        if (!l.conv_kernel.empty()) {
            size_t k = l.conv_k;
            conv_kernels_.push_back((long)backend_->upload(l.conv_kernel.data(), l.conv_kernel.size()));
            conv_k_.push_back(k);
            size_t ring_len = dim * std::max<size_t>(k - 1, 1);
            Buf ring = backend_->alloc(ring_len);
            std::vector<float> zeros(ring_len, 0.0f);
            Buf z = backend_->upload(zeros.data(), ring_len);
            backend_->copy(z, 0, ring, 0, ring_len);
            conv_state_.push_back((long)ring);
        } else {
            conv_kernels_.push_back(-1);
            conv_state_.push_back(-1);
            conv_k_.push_back(0);
        }
    }
    size_t kv = c_.kv_dim(), qd = c_.q_dim();  // :332-354
    x_ = backend_->alloc(dim);
    xb_ = backend_->alloc(dim);
    q_ = backend_->alloc(qd);
    k_ = backend_->alloc(kv);
    v_ = backend_->alloc(kv);
    attn_ = backend_->alloc(qd);
    o_ = backend_->alloc(dim);
    bcx_ = backend_->alloc(3 * dim);
    h_ = backend_->alloc(dim);
    co_ = backend_->alloc(dim);
    cy_ = backend_->alloc(dim);
    gate_ = backend_->alloc(c_.hidden_dim);
    up_ = backend_->alloc(c_.hidden_dim);
    mlp_ = backend_->alloc(dim);
    hidden_ = backend_->alloc(dim);
    att_ = backend_->alloc(c_.n_heads * c_.seq_len);
    logits_ = backend_->alloc(c_.vocab_size);
    logits_host_.assign(c_.vocab_size, 0.0f);
}

// lfm2.rs:380-477
const std::vector<float>& Lfm2::forward(size_t token, size_t pos) {
    size_t dim = c_.dim, hidden = c_.hidden_dim, qd = c_.q_dim(), kv = c_.kv_dim();
    size_t hs = c_.head_dim;
    float eps = c_.rms_eps;
    AttnSpec as{c_.n_heads, c_.kv_mul(), hs, kv, c_.seq_len};
    RopeSpec rs{hs, c_.rope_theta, c_.rope_interleaved};
    size_t positions[1] = {pos};
    Backend& b = *backend_;
    b.embed(token, x_, 0);
    for (size_t l = 0; l < c_.n_layers; l++) {
        const Norms& n = norms_[l];
        b.rms_norm(xb_, x_, n.op, 1, dim, eps);
        if (is_attention_[l]) {
            b.project_qkv(l, xb_, q_, k_, v_, 1);
            if (n.has_q) b.qk_norm(q_, 1, qd, hs, n.q, eps);
            if (n.has_k) b.qk_norm(k_, 1, kv, hs, n.k, eps);
            b.rope(q_, k_, qd, kv, 1, positions, rs);
            b.kv_write(l, positions, k_, v_, 1);
            Window win{0, pos, 0, 0};
            b.attention(q_, attn_, att_, l, &win, 1, as);
            b.project(l, Proj::O, attn_, o_, 1);
            b.add_in_place(x_, o_, dim);
        } else {
            b.project(l, Proj::ConvIn, xb_, bcx_, 1);
            b.mul(h_, 0, bcx_, 0, bcx_, 2 * dim, dim);
            b.conv_decode(co_, h_, (Buf)conv_kernels_[l], (Buf)conv_state_[l], dim, conv_k_[l]);
            b.mul(cy_, 0, bcx_, dim, co_, 0, dim);
            b.project(l, Proj::ConvOut, cy_, o_, 1);
            b.add_in_place(x_, o_, dim);
        }
        b.rms_norm(xb_, x_, n.ffn, 1, dim, eps);
        b.project_gate_up(l, xb_, gate_, up_, 1);
        b.silu_mul(gate_, up_, hidden);
        b.project(l, Proj::Down, gate_, mlp_, 1);
        b.add_in_place(x_, mlp_, dim);
    }
    b.rms_norm(xb_, x_, rms_final_, 1, dim, eps);
    b.logits(xb_, logits_);
    b.read(logits_, logits_host_.data(), logits_host_.size());
    return logits_host_;
}

// lfm2.rs:481-498
const std::vector<float>& Lfm2::prefill(const size_t* tokens, size_t n, size_t start) {
    if (start + n > c_.seq_len) throw std::runtime_error("prefill runs past the context length");
    if (n == 0) return logits_host_;
    std::string st = storage();
    if (st != "f32" && st != "bf16" && st != "q8_0x4") {
        for (size_t i = 0; i < n; i++) forward(tokens[i], start + i);
        return logits_host_;
    }
    prefill_batched(tokens, n, start);
    return logits_host_;
}

// lfm2.rs:501-640
void Lfm2::prefill_batched(const size_t* tokens, size_t n_tok, size_t start) {
    std::vector<size_t> slots, positions;
    std::vector<Window> windows;
    for (size_t i = 0; i < n_tok; i++) {
        slots.push_back(start + i);
        windows.push_back({0, start + i, 0, 0});
    }
    positions = slots;
    size_t dim = c_.dim, hidden = c_.hidden_dim, qd = c_.q_dim(), kv = c_.kv_dim();
    size_t hs = c_.head_dim;
    float eps = c_.rms_eps;
    AttnSpec as{c_.n_heads, c_.kv_mul(), hs, kv, c_.seq_len};
    RopeSpec rs{hs, c_.rope_theta, c_.rope_interleaved};
    Backend& b = *backend_;
    if (!has_prefill_ || pb_.n_tok < n_tok) {  // PrefillBuffers::new lfm2.rs:84-106
        pb_ = PrefillBuffers{n_tok,
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * qd),
                             b.alloc(n_tok * kv),
                             b.alloc(n_tok * kv),
                             b.alloc(n_tok * qd),
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * 3 * dim),
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * dim),
                             b.alloc(n_tok * hidden),
                             b.alloc(n_tok * hidden),
                             b.alloc(n_tok * c_.n_heads * c_.seq_len)};
        has_prefill_ = true;
    }
    for (size_t r = 0; r < n_tok; r++) b.embed(tokens[r], pb_.x, r * dim);
    for (size_t l = 0; l < c_.n_layers; l++) {
        const Norms& n = norms_[l];
        b.rms_norm(pb_.xb, pb_.x, n.op, n_tok, dim, eps);
        if (is_attention_[l]) {
            b.project_qkv(l, pb_.xb, pb_.q, pb_.k, pb_.v, n_tok);
            if (n.has_q) b.qk_norm(pb_.q, n_tok, qd, hs, n.q, eps);
            if (n.has_k) b.qk_norm(pb_.k, n_tok, kv, hs, n.k, eps);
            b.rope(pb_.q, pb_.k, qd, kv, n_tok, positions.data(), rs);
            b.kv_write(l, slots.data(), pb_.k, pb_.v, n_tok);
            b.attention(pb_.q, pb_.attn, pb_.att, l, windows.data(), windows.size(), as);
            b.project(l, Proj::O, pb_.attn, pb_.o, n_tok);
            b.add_in_place(pb_.x, pb_.o, n_tok * dim);
        } else {
            b.project(l, Proj::ConvIn, pb_.xb, pb_.bcx, n_tok);
            for (size_t r = 0; r < n_tok; r++)
                b.mul(pb_.h, r * dim, pb_.bcx, r * 3 * dim, pb_.bcx, r * 3 * dim + 2 * dim, dim);
            size_t k = conv_k_[l];
            b.conv_prefill(pb_.co, pb_.h, (Buf)conv_kernels_[l], n_tok, dim, k);
            if (conv_state_[l] >= 0) {
                size_t take = std::min(n_tok, k - 1);
                b.copy(pb_.h, (n_tok - take) * dim, (Buf)conv_state_[l], (k - 1 - take) * dim, take * dim);
            }
            for (size_t r = 0; r < n_tok; r++)
                b.mul(pb_.cy, r * dim, pb_.bcx, r * 3 * dim + dim, pb_.co, r * dim, dim);
            b.project(l, Proj::ConvOut, pb_.cy, pb_.o, n_tok);
            b.add_in_place(pb_.x, pb_.o, n_tok * dim);
        }
        b.rms_norm(pb_.xb, pb_.x, n.ffn, n_tok, dim, eps);
        b.project_gate_up(l, pb_.xb, pb_.gate, pb_.up, n_tok);
        b.silu_mul(pb_.gate, pb_.up, n_tok * hidden);
        b.project(l, Proj::Down, pb_.gate, pb_.o, n_tok);
        b.add_in_place(pb_.x, pb_.o, n_tok * dim);
    }
    size_t last = (n_tok - 1) * dim;
    b.copy(pb_.x, last, hidden_, 0, dim);
    b.rms_norm(xb_, hidden_, rms_final_, 1, dim, c_.rms_eps);
    b.logits(xb_, logits_);
    b.read(logits_, logits_host_.data(), logits_host_.size());
}

}  // namespace oracle

// TEST INFRASTRUCTURE ONLY. The parity oracle for the kernrt_amd HIP backend.
//
// A plain C++17 restatement of the reference KernRT (Rust) CPU arithmetic on
// the Q8_0 / Q8_0x4 path, compiled with -O2 -ffp-contract=off so that every
// f32 operation rounds where the Rust source rounds: `mul_add` is written as
// fmaf exactly where the reference writes it and nowhere else, `round` is
// roundf (half away from zero) and float->i8 casts saturate (NaN -> 0).
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
// load this code, and only as the checker or the timed CPU baseline. The
// product (kernrt_amd/) never includes or links it.
//
// Every function cites the reference file:line it follows (paths relative to
// the reference repository root). The reference itself cannot be built in
// this image (it is Rust; no cargo/rustc), so this restatement is pinned by
// the reference's own known-answer tests and invariants, by closed forms and
// by brute force; see tests/test_oracle_*.py.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace oracle {

// quant.rs:714, quant.rs:717
constexpr size_t Q8_0_BLOCK = 32;
constexpr size_t Q8_0X4_ROWS = 4;

// quant.rs:722-758
uint16_t f32_to_f16_bits(float value);
// quant.rs:764-769 (normal-only widening; exp==0 widens to 2^-15 * (1+m/1024))
float f16_scale_to_f32(uint16_t bits);
// dot.rs:222-224
float bf16_to_f32(uint16_t bits);
// quant.rs:707-711
uint16_t f32_to_bf16_bits(float value);

// quant.rs:818-825 and quant.rs:831-874
struct Q8Vec {
    std::vector<float> scales;
    std::vector<uint16_t> scales_f16;
    std::vector<int8_t> quants;
    void quantize_into(const float* x, size_t n);
    static Q8Vec quantize(const float* x, size_t n);
};

// quant.rs:113-118 (repr(C), 136 bytes)
struct Q8Block4 {
    uint16_t scales[4];
    int8_t quants[128];
};
static_assert(sizeof(Q8Block4) == 136, "Q8Block4 is 136 bytes");

// quant.rs:502-520
struct Matrix {
    enum Kind { F32, BF16, Q8_0, Q8_0X4 } kind = F32;
    size_t out_dim = 0, in_dim = 0;
    std::vector<float> f32;          // F32
    std::vector<uint16_t> bf16;      // BF16
    std::vector<float> scales;       // Q8_0: one per 32-block, row-major
    std::vector<int8_t> quants;      // Q8_0: out_dim*in_dim
    std::vector<Q8Block4> blocks;    // Q8_0X4: [group][block]

    const Q8Block4& blocks_at(size_t i) const { return blocks[i]; }
    static Matrix from_f32(std::vector<float> data, size_t out, size_t in);
    static Matrix from_bf16_bits(std::vector<uint16_t> bits, size_t out, size_t in);
    // quant.rs:544-557; returns false when in_dim % 32 != 0
    static bool from_f32_q8_0(const std::vector<float>& data, size_t out, size_t in, Matrix* m);
    // quant.rs:124-164; returns false unless in%32==0 and out%4==0
    static bool from_f32_q8_0x4(const std::vector<float>& data, size_t out, size_t in, Matrix* m);

    const char* kind_name() const;  // quant.rs:565-572
    // quant.rs:659-693 (and Q8_0x4::row quant.rs:174-190)
    void decode_row(size_t index, float* out) const;
    std::vector<float> row(size_t index) const;
    // quant.rs:597-612
    std::vector<float> to_f32_tensor() const;
    // quant.rs:620-635
    std::vector<uint16_t> to_bf16_bits() const;
    // quant.rs:198-219 / quant.rs:646-652
    void to_row_major(std::vector<int8_t>* q, std::vector<float>* s) const;
};

// dot.rs:34-45
float dot_q8_0_scalar(const int8_t* a, const float* a_scales, const int8_t* b,
                      const float* b_scales, size_t blocks);
// dot.rs:350-366 (x86 `ops::dot`)
float dot_scalar(const float* a, const float* b, size_t n);
// dot.rs:235-256 (x86 `dot_bf16`)
float dot_bf16_scalar(const uint16_t* a, const float* b, size_t n);
// reference.rs:73-79
float dot_plain(const float* a, const float* b, size_t n);

// quant.rs:23-62
void gemv_into(const Matrix& w, const float* x, float* y);
// quant.rs:66-97 (returns false on a shape error)
bool gemv_q8_0_into(const Matrix& w, const Q8Vec& qx, float* y);
// quant.rs:223-236, x86 fallback
void gemv_q8_0x4(const Matrix& w, const Q8Vec& qx, float* y);
// quant.rs:245-292, portable loop
void gemm_q8_0x4_batched_into(const Matrix& w, const int8_t* quants, const uint16_t* scales_f16,
                              size_t rows, float* y);
// elementwise.rs:81-91
void softmax_in_place(float* x, size_t n);

// ---------------------------------------------------------------------------
// Backends (mod.rs:40-188 types, mod.rs:264-404 trait)

enum class Proj { Q = 0, K = 1, V = 2, O = 3, Gate = 4, Down = 5, Up = 6, ConvIn = 7, ConvOut = 8 };

// formats/llama2c.rs:49-76
struct LayerWeights {
    std::vector<float> rms_att, rms_ffn;
    std::unique_ptr<Matrix> wq, wk, wv, wo, conv_in, conv_out;
    Matrix w1, w2, w3;
    std::vector<float> rms_q, rms_k;  // empty == None
    std::vector<float> conv_kernel;   // [dim, k]; empty == None
    size_t conv_k = 0;
    bool is_attention = true;
    const Matrix* matrix_opt(Proj p) const;  // mod.rs:72-84
};

// mod.rs:131-145
struct ModelWeights {
    Matrix token_embedding;
    std::vector<LayerWeights> layers;
    std::vector<float> rms_final;
    std::unique_ptr<Matrix> wcls;
    const Matrix& classifier() const { return wcls ? *wcls : token_embedding; }
};

struct RopeSpec { size_t head_size; float theta; bool interleaved; };               // mod.rs:149-155
struct AttnSpec { size_t n_heads, kv_mul, head_size, kv_dim, seq_len; };            // mod.rs:158-167
struct KvSpec { size_t n_layers, kv_dim, seq_len; };                                 // mod.rs:170-177
struct Window { size_t att_start, slot, shared_start, shared_end; };                 // mod.rs:181-188

using Buf = size_t;

struct Backend {
    virtual ~Backend() = default;
    virtual const char* name() const = 0;
    virtual const char* storage() const = 0;
    virtual void prepare(std::shared_ptr<const ModelWeights> w, KvSpec kv) = 0;
    virtual Buf alloc(size_t len) = 0;
    virtual Buf upload(const float* data, size_t len) = 0;
    virtual void read(Buf src, float* out, size_t len) = 0;
    virtual void embed(size_t token, Buf out, size_t offset) = 0;
    virtual void copy(Buf src, size_t so, Buf dst, size_t doff, size_t len) = 0;
    virtual void rms_norm(Buf out, Buf x, Buf w, size_t rows, size_t dim, float eps) = 0;
    virtual void qk_norm(Buf v, size_t rows, size_t width, size_t head, Buf w, float eps) = 0;
    virtual void rope(Buf q, Buf k, size_t qw, size_t kvw, size_t rows, const size_t* positions,
                      RopeSpec spec) = 0;
    virtual void project(size_t layer, Proj p, Buf x, Buf y, size_t rows) = 0;
    virtual void project_qkv(size_t layer, Buf x, Buf q, Buf k, Buf v, size_t rows) {
        project(layer, Proj::Q, x, q, rows);
        project(layer, Proj::K, x, k, rows);
        project(layer, Proj::V, x, v, rows);
    }
    virtual void project_gate_up(size_t layer, Buf x, Buf gate, Buf up, size_t rows) {
        project(layer, Proj::Gate, x, gate, rows);
        project(layer, Proj::Up, x, up, rows);
    }
    virtual void kv_write(size_t layer, const size_t* slots, Buf k, Buf v, size_t rows) = 0;
    virtual void attention(Buf q, Buf out, Buf att, size_t layer, const Window* windows,
                           size_t n_windows, AttnSpec spec) = 0;
    virtual void add_in_place(Buf dst, Buf src, size_t len) = 0;
    virtual void mul(Buf out, size_t oo, Buf a, size_t ao, Buf b, size_t bo, size_t len) = 0;
    virtual void conv_prefill(Buf out, Buf x, Buf kernel, size_t rows, size_t dim, size_t k) = 0;
    virtual void conv_decode(Buf out, Buf x, Buf kernel, Buf state, size_t dim, size_t k) = 0;
    virtual void silu_mul(Buf gate, Buf up, size_t len) = 0;
    virtual void logits(Buf x, Buf y) = 0;
};

// cpu.rs:31-129 with prefill_f32 forced off: the f32-widened GEMM path
// (dense.rs:257-342) is a different arithmetic and is not restated, so a Cpu
// built here always runs the int8 path the HIP backend is checked against.
std::unique_ptr<Backend> make_cpu();
// reference.rs:44-415
std::unique_ptr<Backend> make_reference();
// Benchmark set-up only: fill cache slots [0, slots) of every layer with
// N(0, 1) draws (the cpu baseline starts decoding from a pre-filled cache).
void fill_kv(Backend& b, size_t slots, uint64_t seed);
// test set-up: raw values into the key (0) or value (1) cache
void set_kv(Backend& b, int which, size_t offset, const float* data, size_t len);

// arch/llm/llama.rs:26-67
struct Config {
    size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
    float rms_eps, rope_theta;
    bool rope_interleaved;
    size_t head_dim;
    size_t q_dim() const { return n_heads * head_dim; }
    size_t kv_dim() const { return n_kv_heads * head_dim; }
    size_t kv_mul() const { return n_heads / n_kv_heads; }
};

// arch/llm/llama.rs:169-863
class Llama {
public:
    Llama(Config c, std::shared_ptr<const ModelWeights> w, std::unique_ptr<Backend> b);
    const std::vector<float>& forward(size_t token, size_t pos);                    // :786-862
    const std::vector<float>& prefill(const size_t* tokens, size_t n, size_t start);  // :473-492
    std::vector<std::vector<float>> prefill_multi(const std::vector<std::vector<size_t>>& seqs);  // :552-580
    std::vector<std::vector<float>> prefill_shared(const std::vector<size_t>& prefix,
                                                   const std::vector<std::vector<size_t>>& suffixes);  // :603-647
    const char* storage() const { return backend_->storage(); }
    Backend& backend() { return *backend_; }

private:
    struct PrefillRow { size_t token, rope_pos, slot, att_start, sh_start, sh_end; };
    struct PrefillBuffers { size_t n_tok; Buf x, xb, q, k, v, attn, o, gate, up, att; };
    void prefill_batched(const size_t* tokens, size_t n, size_t start);
    void prefill_rows(const std::vector<PrefillRow>& rows);
    std::vector<std::vector<float>> final_hiddens(const std::vector<long>& rows);
    Config c_;
    std::shared_ptr<const ModelWeights> w_;
    std::unique_ptr<Backend> backend_;
    struct Norms { Buf att, ffn, q, k; bool has_q, has_k; };
    std::vector<Norms> norms_;
    Buf rms_final_;
    Buf x_, xb_, q_, k_, v_, attn_, o_, gate_, up_, mlp_, hidden_, att_, logits_;
    std::vector<float> logits_host_;
    bool has_prefill_ = false;
    PrefillBuffers pb_{};
};

// arch/llm/lfm2.rs:118-641
class Lfm2 {
public:
    Lfm2(Config c, std::vector<bool> is_attention, std::shared_ptr<const ModelWeights> w,
         std::unique_ptr<Backend> b);
    const std::vector<float>& forward(size_t token, size_t pos);                    // :380-477
    const std::vector<float>& prefill(const size_t* tokens, size_t n, size_t start);  // :481-498
    const char* storage() const { return backend_->storage(); }
    Backend& backend() { return *backend_; }

private:
    struct PrefillBuffers { size_t n_tok; Buf x, xb, q, k, v, attn, o, bcx, h, co, cy, gate, up, att; };
    void prefill_batched(const size_t* tokens, size_t n, size_t start);
    Config c_;
    std::vector<bool> is_attention_;
    std::vector<size_t> conv_k_;
    std::shared_ptr<const ModelWeights> w_;
    std::unique_ptr<Backend> backend_;
    struct Norms { Buf op, ffn, q, k; bool has_q, has_k; };
    std::vector<Norms> norms_;
    std::vector<long> conv_kernels_, conv_state_;
    Buf rms_final_;
    Buf x_, xb_, q_, k_, v_, attn_, o_, bcx_, h_, co_, cy_, gate_, up_, mlp_, hidden_, att_, logits_;
    std::vector<float> logits_host_;
    bool has_prefill_ = false;
    PrefillBuffers pb_{};
};

// generate.rs:70-77: `max_by(total_cmp)`, which keeps the LAST maximal index.
size_t argmax(const float* v, size_t n);

// tests/backends.rs:41-51 and ops/mod.rs:49-60
std::vector<float> lcg_fill(size_t count, uint64_t seed);

}  // namespace oracle

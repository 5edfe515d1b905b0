// Launchers for the gfx950 kernels of the KernRT HIP backend. Every launcher
// enqueues on the given stream and returns the hipError_t of the launch; the
// host side (backend.cpp) validates shapes before calling any of them.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kr {

// Output-order semantics of a quantized projection (the reference's f32
// epilogue per 32-block; the per-block integer dots are the same for all):
enum Sem {
    // Q8_0x4 project (quant.rs:276-288): slot = fma(f32(isum), f16w(ws)*f16w(xs), slot)
    SEM_FMA_CHAIN = 0,
    // Q8_0 dot (dot.rs:34-45): t[b&3] += (ws*xs)*f32(isum), f32 scales
    SEM_FOUR_PARTIALS_F32 = 1,
    // Q8_0x4 logits on x86 (quant.rs:223-236): as above with f16w(ws)
    SEM_FOUR_PARTIALS_F16 = 2,
};

struct QuantAct {  // one quantized activation batch, row-major
    const int8_t* q;     // [rows][K]
    const float* s;      // [rows][K/32] f32 scales (Q8Vec::scales)
    const uint16_t* h;   // [rows][K/32] f16 bits  (Q8Vec::scales_f16)
};

struct DevMatrix {  // device layout of one Q8 matrix
    int storage;         // KR_STORAGE_Q8_0 or KR_STORAGE_Q8_0X4
    size_t n, k;         // out_dim, in_dim
    int8_t* q;           // [n][k] row-major quants
    void* s;             // [n][k/32]: float (Q8_0) or uint16_t f16 bits (Q8_0x4)
};

hipError_t launch_quantize(hipStream_t st, const float* x, size_t rows, size_t k, size_t x_stride,
                           int8_t* q, float* s, uint16_t* h, bool chain_major = false);

// One launch over up to three matrices with the same in_dim and storage
// (q/k/v, gate/up): output y[i] gets w[i]'s rows, row stride w[i]->n.
hipError_t launch_project_set(hipStream_t st, int sem, const DevMatrix* const* w, float* const* y, int count,
                              QuantAct x, size_t rows, int32_t* dbg_block_dots);

// Fused decode/prefill steps (same arithmetic as the separate ops):
// x += add (when add != null), out = rms_norm(x) and its Q8 quantization.
// add_planes 4: `add` holds a chain-split projection's four partial-sum planes;
// chain_major: the Q8 blocks in chain-major order (for launch_gemm_q8_cs)
hipError_t launch_add_rms_quant(hipStream_t st, float* x, const float* add, const float* w, float* out,
                                size_t rows, size_t dim, float eps, int8_t* q, float* s, uint16_t* h,
                                int add_planes = 1, bool chain_major = false);
// g = silu(g) * u and its Q8 quantization, rows of `width`
hipError_t launch_silu_quant(hipStream_t st, float* g, const float* u, size_t rows, size_t width, int8_t* q,
                             float* s, uint16_t* h);
// RoPE of q and k, then k and v into the cache at slots[row]
hipError_t launch_rope_kv(hipStream_t st, float* q, float* k, const float* v, size_t qw, size_t kvw,
                          size_t rows, const uint32_t* positions, const uint32_t* slots, const float2* table,
                          size_t head_size, int interleaved, float* kc, float* vc, size_t layer, size_t seq_len);
// per-head RMSNorm of q (weight wq) and k (wk), then launch_rope_kv's work, in one launch
hipError_t launch_qk_norm_rope_kv(hipStream_t st, float* q, float* k, const float* v, size_t qw, size_t kvw,
                                  size_t rows, const float* wq, const float* wk, float eps,
                                  const uint32_t* positions, const uint32_t* slots, const float2* table,
                                  size_t head_size, int interleaved, float* kc, float* vc, size_t layer,
                                  size_t seq_len);

// y[m*ldy + n] for m < rows. Uses the GEMV path (rows <= 4) or the MFMA GEMM.
// One decode row (M = 1) of 1-3 projections with the producer of their input
// fused in front: pro_kind 1 = x (+= add) -> rms_norm(w, eps) -> Q8 (the
// updated x row goes to x_out when non-null), 3 = Q8 of the f32 row a.
// One decode row of gate/up with the producer in front (x (+= add) ->
// rms_norm(norm_w, eps) -> Q8, the updated x row to x_out when non-null) and
// h = silu(gate) * up behind, quantized into (hq, hs, hh) for the down
// projection; h itself goes to hf when non-null. Needs swiglu_fusable.
bool swiglu_fusable(const DevMatrix& gate, const DevMatrix& up);
// Prefill gate/up of Q8_0 matrices with SiLU(gate) * up and its Q8 blocks as
// the GEMM's epilogue: h's quants / f32 scales / f16 scale bits [rows][n]
// from the quantized rows x (one launch for gate/up + silu_quant).
// The chain-split Q8_0 GEMM (gemm.hip): `cm` is a chain-major copy (launch_chain_major),
// x chain-major too; y4 receives the four partial-sum planes [4][rows][cm.n].
hipError_t launch_chain_major(hipStream_t st, const DevMatrix& m, int8_t* cq, float* cs);
// The q/k/v GEMM with RoPE (head_dim 64, half-split layout) and kv_write as its
// epilogue (gemm.hip): q rotated into yq, k rotated and v into kc / vc (the
// layer's cache) at each row's slot.
bool qkv_rope_q8_ok(const DevMatrix& q, const DevMatrix& k, const DevMatrix& v, size_t rows);
hipError_t launch_qkv_rope_q8(hipStream_t st, const DevMatrix& q, const DevMatrix& k, const DevMatrix& v, QuantAct x,
                              size_t rows, float* yq, const uint32_t* pos, const uint32_t* slots, const float2* tab,
                              float* kc, float* vc);
hipError_t launch_gemm_q8_cs(hipStream_t st, const DevMatrix& cm, QuantAct x, size_t rows, float* y4);
hipError_t launch_gate_up_silu_q8(hipStream_t st, const DevMatrix& gate, const DevMatrix& up, QuantAct x, size_t rows,
                                  int8_t* hq, float* hs, uint16_t* hh, bool chain_major = false);
hipError_t launch_gate_up_swiglu(hipStream_t st, int sem, const DevMatrix& gate, const DevMatrix& up, const float* x,
                                 const float* add, const float* norm_w, float* x_out, float eps, int8_t* hq,
                                 float* hs, uint16_t* hh, float* hf);
hipError_t launch_project_pro(hipStream_t st, int sem, const DevMatrix* const* w, float* const* y, int count,
                              int pro_kind, const float* a, const float* b, const float* norm_w, float* x_out,
                              float eps);
hipError_t launch_project(hipStream_t st, int sem, const DevMatrix& w, QuantAct x, size_t rows,
                          float* y, size_t ldy, int32_t* dbg_block_dots);

hipError_t launch_rms_norm(hipStream_t st, float* out, const float* x, const float* w, size_t rows,
                           size_t dim, float eps);
// per-head RMSNorm of the rows of v (width = heads * head); with v2 non-null
// also those of v2 (width2, weight w2) in the same launch
hipError_t launch_qk_norm(hipStream_t st, float* v, size_t rows, size_t width, size_t head,
                          const float* w, float eps, float* v2 = nullptr, size_t width2 = 0,
                          const float* w2 = nullptr);
// table: [n_pos][head_size/2] of (cos, sin)
hipError_t launch_rope(hipStream_t st, float* q, float* k, size_t qw, size_t kvw, size_t rows,
                       const uint32_t* positions, const float2* table, size_t head_size, int interleaved);
hipError_t launch_kv_write(hipStream_t st, float* kc, float* vc, size_t layer, size_t seq_len,
                           size_t kv_dim, const uint32_t* slots, const float* k, const float* v,
                           size_t rows);
struct DevWindow { uint32_t att_start, slot, shared_start, shared_end; };
hipError_t launch_attention(hipStream_t st, const float* q, float* out, float* att, const float* kc,
                            const float* vc, size_t layer, const DevWindow* windows, size_t n_rows,
                            size_t max_count, size_t n_heads, size_t kv_mul, size_t head_size,
                            size_t kv_dim, size_t seq_len, float scale, int8_t* qo = nullptr,
                            float* so = nullptr, uint16_t* ho = nullptr, const DevWindow* host_windows = nullptr,
                            float* mx_scratch = nullptr, bool keep_att = true);
// Prefill attention on the matrix core (attn_mx.hip): whether a launch can
// take it (head size 64 or 128, a longest window of 1024 to 4096 positions,
// every block of 32 / G rows sharing one window layout), and the launch.
bool attention_mx_ok(const DevWindow* w, size_t n_rows, size_t max_count, size_t kv_mul, size_t hs);
// `scratch` holds 2 n_rows n_heads floats (each pair's max and sum).
hipError_t launch_attention_mx(hipStream_t st, const float* q, float* out, float* att, const float* kc,
                               const float* vc, size_t layer, const DevWindow* windows, size_t n_rows,
                               size_t max_count, size_t n_heads, size_t kv_mul, size_t hs, size_t kv_dim,
                               size_t seq_len, float scale, int8_t* qo, float* so, uint16_t* ho, float* scratch,
                               bool keep_att = true);
// Decode attention of one row in two launches (scores by 64-row chunks with
// RoPE and the kv_write of k/v folded in, and the per-head q / k RMSNorm
// where qnw / knw are given, then softmax + V by head slices of 4 dims);
// `scratch` holds
// attention_split_scratch(n_heads, seq_len) floats.
bool attention_split_ok(size_t max_count, size_t kv_mul, size_t hs);
// launch_attention_split_rows's geometry check (k_attn_softmax_v_rows).
bool attention_split_rows_ok(size_t max_count, size_t kv_mul, size_t hs);
size_t attention_split_scratch(size_t n_heads, size_t seq_len);
hipError_t launch_attention_split(hipStream_t st, const float* q, const float* k, const float* v, float* out,
                                  float* att, float* kc, float* vc, size_t layer, const DevWindow* window,
                                  const uint32_t* pos, const float2* table, int interleaved, size_t max_count,
                                  size_t n_heads, size_t kv_mul, size_t hs, size_t kv_dim, size_t seq_len,
                                  float scale, float* scratch, const float* qnw = nullptr,
                                  const float* knw = nullptr, float eps = 0.0f);
// The same two launches for many rows with windows of their own (batched
// decode): q rows already rotated, keys already in the cache; `scratch`
// holds n_rows * attention_split_scratch(n_heads, seq_len) floats. keep_att
// false leaves `att` unwritten; qo/so/ho (head size a multiple of 32) take
// the output rows' Q8 blocks as well.
hipError_t launch_attention_split_rows(hipStream_t st, const float* q, float* out, float* att, const float* kc,
                                       const float* vc, size_t layer, const DevWindow* windows, size_t n_rows,
                                       size_t max_count, size_t n_heads, size_t kv_mul, size_t hs, size_t kv_dim,
                                       size_t seq_len, float scale, float* scratch, bool keep_att = true,
                                       int8_t* qo = nullptr, float* so = nullptr, uint16_t* ho = nullptr);
// whether the rows' windows let launch_attention use its block-of-rows
// (prefill) kernel: each block of rows shares att_start and the shared range
bool attention_rows_uniform(const DevWindow* host_windows, size_t n_rows, size_t max_count, size_t kv_mul,
                            size_t hs);
hipError_t launch_add(hipStream_t st, float* dst, const float* src, size_t n);
hipError_t launch_add_planes(hipStream_t st, float* dst, const float* planes, size_t n);
hipError_t launch_mul(hipStream_t st, float* out, const float* a, const float* b, size_t n,
                      int sequential);
// o[r os + i] = a[r as + i] * b[r bs + i] for r < rows, i < n (no overlap of o with a or b)
hipError_t launch_mul_rows(hipStream_t st, float* o, size_t os, const float* a, size_t as, const float* b, size_t bs,
                           size_t rows, size_t n);
hipError_t launch_copy(hipStream_t st, float* dst, const float* src, size_t n);
// reads n floats (n % 4 == 0) and discards them, cpl (1, 2, 4, 8) 16-byte
// loads per lane per round, on `workgroups` workgroups of 256 (0: one round
// each); `sink` is never written in practice
hipError_t launch_serial_sum_probe(hipStream_t st, const float* x, size_t n, size_t count, int waves,
                                   uint32_t* out);
hipError_t launch_stream_read(hipStream_t st, const float* p, size_t n, int* sink, int cpl = 2,
                              size_t workgroups = 0);
hipError_t launch_silu_mul(hipStream_t st, float* g, const float* u, size_t n);
// causal depthwise conv of rows of x; history before row 0 is zero padding
// (state null) or the ring `state` of k - 1 rows, oldest first
hipError_t launch_conv_prefill(hipStream_t st, float* out, const float* x, const float* kernel,
                               size_t rows, size_t dim, size_t k, const float* state = nullptr);
// the ring after `rows` rows of x have entered it one at a time (k <= 16)
hipError_t launch_conv_ring_advance(hipStream_t st, float* state, const float* x, size_t rows, size_t dim,
                                    size_t k);
// y = C * conv(B * x) for one decode row, bcx = [B | C | x] (3 * dim), the
// conv state shifted in place
hipError_t launch_conv_block_decode(hipStream_t st, float* y, const float* bcx, const float* kern, float* state,
                                    size_t dim, size_t k);
hipError_t launch_conv_decode(hipStream_t st, float* out, const float* x, const float* kernel,
                              float* state, size_t dim, size_t k);
// token from `token_dev` when non-null, else `token`
// rows 0..n-1 of out (row stride e.k) get the embeddings of tokens_dev[0..n-1]
hipError_t launch_embed_rows(hipStream_t st, const DevMatrix& e, const uint32_t* tokens_dev, size_t n, float* out);
hipError_t launch_embed(hipStream_t st, const DevMatrix& e, size_t token, const uint32_t* token_dev,
                        float* out);
hipError_t launch_argmax(hipStream_t st, const float* x, size_t n, uint32_t* out);
hipError_t launch_greedy_step(hipStream_t st, const float* logits, size_t n, uint32_t* step, uint32_t* ring,
                              size_t ring_len);
hipError_t launch_synthetic_q8(hipStream_t st, const DevMatrix& m, uint64_t seed, float stddev);
// rows [row0, row0 + rows) of m quantized from f32 values or bf16 bits (src holds those rows only)
hipError_t launch_quant_weights(hipStream_t st, const DevMatrix& m, size_t row0, size_t rows, const void* src,
                                int bf16);
hipError_t launch_synthetic_normal(hipStream_t st, float* out, size_t n, uint64_t seed);
// int8 MFMA throughput probe: blocks x 256 threads, `iters` rounds; *ops = int8 ops issued;
// sink holds blocks * 256 ints
hipError_t launch_mfma_spin(hipStream_t st, int kind, int* sink, size_t blocks, uint32_t iters, double* ops);
// One f32 matrix instruction (v_mfma_f32_32x32x1_2b_f32) per group of 64
// lanes on given operands, for exactness checks: a, b [groups][64], c and out
// [groups][32][64] (register v of lane l)
hipError_t launch_mfma_f32_probe(hipStream_t st, const float* a, const float* b, const float* c, float* out,
                                 size_t groups);
// the f32 values launch_synthetic_q8 quantizes, element i of the flattened matrix
hipError_t launch_synthetic_values(hipStream_t st, float* out, size_t n, uint64_t seed, float stddev);
// counts Q8_0x4 blocks whose max |q| is neither 0 nor 127
hipError_t launch_requant_check(hipStream_t st, const DevMatrix& m, unsigned int* counter);
// x86 `gemv_q8_0x4` re-quantization of every row into a Q8_0 matrix (quant.rs:232-235)
hipError_t launch_requantize(hipStream_t st, const DevMatrix& src, const DevMatrix& dst);

}  // namespace kr

// Backend entry points used by the in-library model driver (llm.cpp) but not
// part of the public C ABI: decode-step variants whose per-token scalars
// (token id, position) live in device memory, so a whole decode step is a
// fixed launch sequence that can be captured once in a HIP graph and
// replayed per token.
//
// Device step record (uint32_t[8]):
//   [0] token  [1] att_start  [2] slot == position  [3] shared_start
//   [4] shared_end  [5] step index into the token ring  [6..7] unused
// so &s[1] is a window {att_start, slot, shared_start, shared_end}, &s[2] the
// position and the KV slot, &s[0] the token.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/kernrt_hip.h"

namespace kri {

hipStream_t stream(kr_ctx* c);
int set_error(kr_ctx* c, int code, const char* msg);
int device_u32(kr_ctx* c, size_t n, uint32_t** out);
void device_free(void* p);
uint32_t* token_ring(kr_ctx* c);
// changes whenever the backend reallocates a buffer that captured kernels may
// reference; a cached graph from an older epoch must be re-captured
uint64_t epoch(kr_ctx* c);
size_t token_ring_len();

int embed_dev(kr_ctx* c, const uint32_t* token_dev, kr_buf out, size_t offset);
// rows 0..n-1 of out get the embeddings of tokens[0..n-1] (one launch)
int embed_rows(kr_ctx* c, const size_t* tokens, size_t n, kr_buf out);
int rope_dev(kr_ctx* c, kr_buf q, kr_buf k, size_t qw, size_t kvw, const uint32_t* pos_dev,
             const kr_rope_spec* spec);
int kv_write_dev(kr_ctx* c, size_t layer, const uint32_t* slot_dev, kr_buf k, kr_buf v);
int attention_dev(kr_ctx* c, kr_buf q, kr_buf out, kr_buf att, size_t layer, const uint32_t* window_dev,
                  const kr_attn_spec* spec);
// argmax of logits -> s[0] and ring[s[5]]; then s[2] += 1, s[5] += 1
int greedy_step(kr_ctx* c, kr_buf logits, size_t len, uint32_t* step);

// Fused driver steps. Each leaves the Q8 quantization of its output rows in
// the backend's activation workspace, which project_q / logits_q consume.
// x += add (add may be KR_NO_BUF), out = rms_norm(x, w), quantize(out)
int norm_quant(kr_ctx* c, kr_buf x, kr_buf add, int add_planes, kr_buf w, kr_buf out, size_t rows, size_t dim,
               float eps, bool chain_major = false);
// dst += ((p0 + p1) + p2) + p3 over the four planes of a chain-split projection
int add_planes(kr_ctx* c, kr_buf dst, kr_buf planes, size_t len);
// projections of the quantized workspace rows; one launch when they share in_dim and storage
int project_q(kr_ctx* c, size_t layer, const int* projs, const kr_buf* ys, int n, size_t rows);
// out[oo + r os + i] = a[ao + r as + i] * b[bo + r bs + i], r < rows, i < n, one launch
// (out must not be a or b)
int mul_rows(kr_ctx* c, kr_buf out, size_t oo, size_t os, kr_buf a, size_t ao, size_t as, kr_buf b, size_t bo,
             size_t bs, size_t rows, size_t n);
// gate = silu(gate) * up, quantized
int silu_quant(kr_ctx* c, kr_buf gate, kr_buf up, size_t rows, size_t width);
// prefill FFN after the norm's quantization: gate/up + SiLU * up + Q8 in one
// GEMM launch, then down into `out` (Q8_0 gate/up, rows >= 8)
bool ffn_swiglu_ok(kr_ctx* c, size_t layer, size_t rows);
// max_planes 4: the down projection may run chain-split and leave its four
// partial-sum planes in `out` (room for 4 x rows x dim); *planes says which
int ffn_swiglu_down(kr_ctx* c, size_t layer, size_t rows, kr_buf out, int max_planes, int* planes);
// prefill q/k/v after the norm's quantization with RoPE (head_dim 64, the
// half-split layout, no q/k norm) and kv_write as the GEMM's epilogue: q
// rotated into `q`, k and v into the layer's cache (the k and v buffers are
// not written)
bool qkv_rope_ok(kr_ctx* c, size_t layer, size_t rows, const kr_rope_spec* spec);
int project_qkv_rope(kr_ctx* c, size_t layer, kr_buf q, size_t rows, const size_t* pos_host, const size_t* slot_host,
                     const kr_rope_spec* spec);
// rope of q and k, then k and v into the cache; positions and slots from the
// host (pos_host/slot_host) or one device position (pos_dev, rows == 1).
// With the weights nq and nk, the per-head RMSNorms of q and k (eps) come
// first, in the same launch.
int rope_kv(kr_ctx* c, kr_buf q, kr_buf k, kr_buf v, size_t qw, size_t kvw, size_t rows, const size_t* pos_host,
            const size_t* slot_host, const uint32_t* pos_dev, size_t layer, const kr_rope_spec* spec,
            kr_buf nq = KR_NO_BUF, kr_buf nk = KR_NO_BUF, float eps = 0.0f);
// attention whose output rows are also quantized; windows from the host, or
// one device window (window_dev, n == 1). keep_att false: the prefill forms
// may leave `att` without the final probabilities (the driver never reads
// its scratch rows back); every output is unchanged
int attention_quant(kr_ctx* c, kr_buf q, kr_buf out, kr_buf att, size_t layer, const kr_window* windows,
                    size_t n, const uint32_t* window_dev, const kr_attn_spec* spec, bool keep_att = true);
// the classifier over the quantized workspace row
int logits_q(kr_ctx* c, kr_buf y);
// the classifier over the first `rows` quantized workspace rows -> y [rows][vocab]
int logits_rows(kr_ctx* c, kr_buf y, size_t rows);

// One decode row with the producer of the projection input fused into the
// projection launch (results identical to the separate steps above):
// whether a row of width k can take this path
bool pro_fusable(size_t k);
// x_out = x + add (add may be KR_NO_BUF), then the projections of
// Q8(rms_norm(x_out, w)); x_out must not be x
int norm_project(kr_ctx* c, size_t layer, const int* projs, const kr_buf* ys, int n, kr_buf x, kr_buf add, kr_buf w,
                 kr_buf x_out, size_t dim, float eps);
// gate/up of Q8(rms_norm(x + add, w)) with Q8(silu(gate) * up) into the
// activation workspace (h = silu(gate) * up to `h`); x_out must not be x
bool swiglu_ok(kr_ctx* c, size_t layer, size_t dim);
int norm_swiglu(kr_ctx* c, size_t layer, kr_buf x, kr_buf add, kr_buf w, kr_buf x_out, kr_buf h, size_t dim,
                float eps);
// kr_qk_norm of q and of k in one launch
int qk_norm_pair(kr_ctx* c, kr_buf q, kr_buf k, size_t rows, size_t q_width, size_t k_width, size_t head,
                 kr_buf wq, kr_buf wk, float eps);
// y = C * conv(B * x) of one LFM2 decode row, bcx = [B | C | x]
int conv_block_decode(kr_ctx* c, kr_buf y, kr_buf bcx, kr_buf kernel, kr_buf state, size_t dim, size_t k);
// conv of `rows` rows of x with the ring as their history, then the ring
// advanced past them: the values of `rows` conv_decode steps in one launch
int conv_prefill_stepped(kr_ctx* c, kr_buf out, kr_buf x, kr_buf kernel, kr_buf state, size_t rows, size_t dim,
                         size_t k);
// the projection of Q8(x) (x one f32 row of `width`)
int quant_project(kr_ctx* c, size_t layer, int proj, kr_buf x, kr_buf y, size_t width);

// Decode attention of one row as two launches that spread the cache reads
// over many CUs, with rope of q and k and the kv_write of k and v folded in:
// the same values as rope_kv + attention. Whether it applies to `spec` for
// windows of up to max_count positions:
bool split_attention_ok(kr_ctx* c, const kr_attn_spec* spec, size_t max_count);
// window {0, pos, 0, 0} and position from the host (pos_host), or from the
// device step record (step_dev: window at step[1..4], position at step[2],
// the window at most dev_max_count positions: the launch is sized for it)
// nq / nk: per-head RMSNorm weights of q / k applied before the rotation
// (either may be KR_NO_BUF)
int rope_attention(kr_ctx* c, kr_buf q, kr_buf k, kr_buf v, kr_buf out, kr_buf att, size_t layer, size_t pos_host,
                   const uint32_t* step_dev, const kr_attn_spec* spec, const kr_rope_spec* rope,
                   size_t dev_max_count, kr_buf nq = KR_NO_BUF, kr_buf nk = KR_NO_BUF, float eps = 0.0f);

}  // namespace kri

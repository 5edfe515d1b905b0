/*
 * kernrt_llm.h — the model drivers above the backend seam, in C++ with a C
 * ABI: the host-side mirror of the reference's `Llama`
 * (src/arch/llm/llama.rs:169-863) and `Lfm2` (src/arch/llm/lfm2.rs:118-641),
 * driving a `kr_ctx` through the calls of include/kernrt_hip.h exactly as the
 * reference drivers drive `dyn Backend`.
 *
 * The reference is Rust; with no Rust toolchain in this build's image the
 * driver is C++. A Rust `backends/hip.rs` arm over kernrt_hip.h forwards
 * each `Backend` method to the kr_* call of the same name and arguments.
 */
#ifndef KERNRT_LLM_H
#define KERNRT_LLM_H

#include <stddef.h>
#include <stdint.h>

#include "kernrt_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct krl_model krl_model;

/* arch/llm/llama.rs:26-67 `Config`. */
typedef struct {
    size_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
    float rms_eps, rope_theta;
    int rope_interleaved;
    size_t head_dim;
} krl_config;

/* The small f32 tensors of one `LayerWeights` (formats/llama2c.rs:49-76);
 * the matrices are bound on the backend with kr_bind_proj beforehand. */
typedef struct {
    const float* rms_att;     /* [dim] (LFM2: operator_norm) */
    const float* rms_ffn;     /* [dim] */
    const float* rms_q;       /* [head_dim] or NULL */
    const float* rms_k;       /* [head_dim] or NULL */
    const float* conv_kernel; /* LFM2 conv layers: [dim, conv_k]; else NULL */
    size_t conv_k;
    int is_attention;
} krl_layer;

typedef struct {
    const krl_layer* layers; /* n_layers entries */
    const float* rms_final;  /* [dim] */
} krl_weights;

/* Llama::with_backend (llama.rs:364-415) / Lfm2::with_backend (lfm2.rs:276-366):
 * calls kr_prepare on `backend` (matrices must be bound), uploads the norms,
 * allocates the decode state. The model borrows `backend`; close it after
 * krl_free. */
int krl_llama_new(kr_ctx* backend, const krl_config* cfg, const krl_weights* w, krl_model** out);
int krl_lfm2_new(kr_ctx* backend, const krl_config* cfg, const krl_weights* w, krl_model** out);
void krl_free(krl_model* m);
const char* krl_last_error(const krl_model* m);

/* forward(token, pos) -> logits (llama.rs:786-862, lfm2.rs:380-477). */
int krl_forward(krl_model* m, size_t token, size_t pos, float* logits);
/* prefill(tokens, start) -> logits of the last row (llama.rs:473-492,
 * lfm2.rs:481-498). Every storage runs batched here. For a Q8_0 model the
 * reference loops forward() token by token instead; the batch gives that
 * loop's values: Llama rows are independent apart from causal attention
 * over the same cache, and an LFM2's conv layers take their history from the
 * conv ring and advance it as the token loop would (so a chunked prefill or
 * a prefill after decoding continues the ring). For q8_0x4 the LFM2 conv is
 * the reference's batched one: zero history before the first row, then the
 * last k - 1 rows copied into the ring's tail (lfm2.rs:587-603). */
int krl_prefill(krl_model* m, const size_t* tokens, size_t n, size_t start, float* logits);
/* prefill_multi / prefill_shared (llama.rs:552-647): sequences flattened,
 * `lens[i]` tokens each; one final-normed hidden row [dim] per sequence. */
int krl_prefill_multi(krl_model* m, const size_t* tokens, const size_t* lens, size_t n_seq, float* hiddens);
int krl_prefill_shared(krl_model* m, const size_t* prefix, size_t n_prefix, const size_t* tokens,
                       const size_t* lens, size_t n_seq, float* hiddens);

/* One decode step for n_seq independent sequences that share the model and
 * the cache, the batched shape of forward() (no counterpart in the
 * reference, whose forward and logits take one row; the rows are laid out as
 * prefill_multi lays out its sequences, llama.rs:552-580): row s feeds
 * tokens[s] at RoPE position rope_pos[s] into cache slot slots[s] and
 * attends over slots att_start[s] ..= slots[s]. Writes logits
 * [n_seq][vocab_size] (unless `logits` is null: they then stay on the
 * device); row s equals what forward() gives for that sequence alone. Llama
 * models only. */
int krl_decode_batch(krl_model* m, const size_t* tokens, const size_t* rope_pos, const size_t* slots,
                     const size_t* att_start, size_t n_seq, float* logits);

/* Greedy decoding of `n_steps` tokens after `token` at position `pos`, with
 * the argmax (generate.rs:70-77 tie rule) on the device. Each step is the
 * forward pass with its token and position read from device memory; with
 * `use_graph` the step is captured once as a HIP graph and replayed.
 * out_tokens[i] is the token chosen at step i (its logits came from position
 * pos + i). */
int krl_generate_greedy(krl_model* m, size_t token, size_t pos, size_t n_steps, size_t* out_tokens,
                        int use_graph);

#ifdef __cplusplus
}
#endif

#endif /* KERNRT_LLM_H */

/*
 * kernrt_hip.h — C ABI of libkernrt_hip.so, the MI355X (gfx950) backend for
 * KernRT's `Backend` trait (reference: src/backends/mod.rs:264-404).
 *
 * One `kr_ctx` is one backend instance: one device, one in-order HIP stream,
 * its activation buffers, its weights and its key/value cache. Calls are
 * stream-ordered and may return before the device has finished; `kr_read` is
 * the barrier (mod.rs:262-282). A context is used from one thread at a time
 * (the trait is `Send`, not `Sync`).
 *
 * Every entry returns KR_OK or an error code; `kr_last_error` gives the text.
 * The reference trait panics on misuse (cpu.rs:134, :366); a binding maps a
 * non-zero status to that panic. Only `kr_open` distinguishes "no device"
 * (KR_ERR_NO_DEVICE, detail "no HIP device ...") from other failures, which is
 * what `BackendError::detail` carries (mod.rs:190-213).
 *
 * Plain C types only; host slices (positions, slots, windows) are copied
 * before the call returns, so the caller may reuse them immediately.
 */
#ifndef KERNRT_HIP_H
#define KERNRT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kr_ctx kr_ctx;
/* A handle to activation memory (mod.rs:40-42 `Buf`). */
typedef uint32_t kr_buf;
/* A device-resident weight matrix (one `Matrix`, quant.rs:502-520). */
typedef uint32_t kr_mat;
#define KR_NO_MAT ((kr_mat)0xffffffffu)
#define KR_NO_BUF ((kr_buf)0xffffffffu)

enum {
    KR_OK = 0,
    KR_ERR_NO_DEVICE = 1, /* open: no usable gfx950 device */
    KR_ERR_INVALID = 2,   /* bad handle, shape or argument */
    KR_ERR_HIP = 3,       /* a HIP runtime call failed */
    KR_ERR_OOM = 4,       /* device allocation failed */
    KR_ERR_STATE = 5      /* call out of order (e.g. compute before prepare) */
};

/* Projection index, `Proj::index` (mod.rs:100-112). */
enum {
    KR_PROJ_Q = 0, KR_PROJ_K = 1, KR_PROJ_V = 2, KR_PROJ_O = 3, KR_PROJ_GATE = 4,
    KR_PROJ_DOWN = 5, KR_PROJ_UP = 6, KR_PROJ_CONV_IN = 7, KR_PROJ_CONV_OUT = 8
};

/* Weight storage kinds (`Matrix` variants, quant.rs:502-520). */
enum { KR_STORAGE_Q8_0 = 2, KR_STORAGE_Q8_0X4 = 3 };

/* `Window` (mod.rs:181-188): own range [att_start, slot], plus the shared
 * range [shared_start, shared_end) scored first. */
typedef struct {
    size_t att_start, slot, shared_start, shared_end;
} kr_window;

/* `AttnSpec` (mod.rs:158-167). */
typedef struct {
    size_t n_heads, kv_mul, head_size, kv_dim, seq_len;
} kr_attn_spec;

/* `RopeSpec` (mod.rs:149-155). */
typedef struct {
    size_t head_size;
    float theta;
    int interleaved;
} kr_rope_spec;

/* ---- lifetime (backends::open, mod.rs:228-244; Backend::name/storage :266-269) */
int kr_open(int device, kr_ctx** out, char* detail, size_t detail_len);
void kr_close(kr_ctx* ctx);
const char* kr_last_error(const kr_ctx* ctx);
const char* kr_name(const kr_ctx* ctx);    /* "hip" */
const char* kr_storage(const kr_ctx* ctx); /* the embedding's storage, like cpu.rs:196 */
int kr_device_name(const kr_ctx* ctx, char* out, size_t len);

/* ---- weights: the material `prepare` receives (mod.rs:271-272, 131-145) */
/* Matrix::Q8_0 (quant.rs:512-517): row-major int8 quants, one f32 scale per 32-block. */
int kr_matrix_q8_0(kr_ctx* ctx, size_t out_dim, size_t in_dim, const int8_t* quants,
                   const float* scales, kr_mat* out);
/* Matrix::Q8_0x4 (quant.rs:103-118): (out_dim/4)*(in_dim/32) packed 136-byte
 * blocks {u16 scales[4]; i8 quants[128]}, de-interleaved on upload. */
int kr_matrix_q8_0x4(kr_ctx* ctx, size_t out_dim, size_t in_dim, const void* blocks, kr_mat* out);
/* Synthetic weights for benchmarks: N(0, stddev) from a counter-based
 * generator on the device, quantized with the same arithmetic as
 * Matrix::from_f32_q8_0 / Q8_0x4::from_f32 (quant.rs:544-557, 124-164). */
int kr_matrix_synthetic(kr_ctx* ctx, int storage, size_t out_dim, size_t in_dim, uint64_t seed,
                        float stddev, kr_mat* out);
/* The f32 values kr_matrix_synthetic quantizes for (seed, stddev): element i
 * of the flattened [out_dim, in_dim] matrix into out[i], i < n -- so a checker
 * can quantize them the reference's way and compare with kr_matrix_read. */
int kr_synthetic_values(kr_ctx* ctx, kr_buf out, size_t n, uint64_t seed, float stddev);
/* Checkpoint weights quantized on the device: `data` holds out_dim rows of
 * in_dim values, f32 (KR_SRC_F32) or bf16 bit patterns (KR_SRC_BF16, widened
 * exactly as hf.rs:93-103 does), row-major, in host memory; the result is the
 * matrix Matrix::from_f32_q8_0 (quant.rs:544-557) or Q8_0x4::from_f32
 * (quant.rs:124-164) would build from those values, as matrix_from_raw
 * (hf.rs:151-200) asks for it. Q8_0x4 needs out_dim % 4 == 0. */
#define KR_SRC_F32 0
#define KR_SRC_BF16 1
int kr_matrix_quantize(kr_ctx* ctx, int storage, int src_kind, const void* data, size_t out_dim, size_t in_dim,
                       kr_mat* out);
int kr_matrix_free(kr_ctx* ctx, kr_mat m);

/* Bind matrices into the model layout, then `prepare` (mod.rs:272). */
int kr_bind_embedding(kr_ctx* ctx, kr_mat m);
int kr_bind_classifier(kr_ctx* ctx, kr_mat m); /* KR_NO_MAT: tied to the embedding */
int kr_bind_proj(kr_ctx* ctx, size_t layer, int proj, kr_mat m);
int kr_prepare(kr_ctx* ctx, size_t n_layers, size_t kv_dim, size_t seq_len); /* KvSpec mod.rs:170-177 */

/* ---- memory (mod.rs:274-282) */
int kr_alloc(kr_ctx* ctx, size_t len, kr_buf* out);                   /* Backend::alloc, zeroed */
int kr_upload(kr_ctx* ctx, const float* data, size_t len, kr_buf* out); /* Backend::upload */
int kr_read(kr_ctx* ctx, kr_buf src, float* out, size_t len);          /* Backend::read: the barrier */

/* ---- ops (mod.rs:284-403) */
int kr_embed(kr_ctx* ctx, size_t token, kr_buf out, size_t offset);                     /* :285 */
int kr_copy(kr_ctx* ctx, kr_buf src, size_t src_offset, kr_buf dst, size_t dst_offset,  /* :288 */
            size_t len);
int kr_rms_norm(kr_ctx* ctx, kr_buf out, kr_buf x, kr_buf weight, size_t rows, size_t dim,  /* :291 */
                float eps);
int kr_qk_norm(kr_ctx* ctx, kr_buf v, size_t rows, size_t width, size_t head_size,          /* :294-302 */
               kr_buf weight, float eps);
int kr_rope(kr_ctx* ctx, kr_buf q, kr_buf k, size_t q_width, size_t kv_width, size_t rows,  /* :306-315 */
            const size_t* positions, const kr_rope_spec* spec);
int kr_project(kr_ctx* ctx, size_t layer, int proj, kr_buf x, kr_buf y, size_t rows);     /* :318 */
int kr_project_qkv(kr_ctx* ctx, size_t layer, kr_buf x, kr_buf q, kr_buf k, kr_buf v,     /* :326-330 */
                   size_t rows);
int kr_project_gate_up(kr_ctx* ctx, size_t layer, kr_buf x, kr_buf gate, kr_buf up,       /* :334-337 */
                       size_t rows);
int kr_kv_write(kr_ctx* ctx, size_t layer, const size_t* slots, kr_buf k, kr_buf v,       /* :344 */
                size_t rows);
int kr_attention(kr_ctx* ctx, kr_buf q, kr_buf out, kr_buf att, size_t layer,             /* :351-359 */
                 const kr_window* windows, size_t n_windows, const kr_attn_spec* spec);
int kr_add_in_place(kr_ctx* ctx, kr_buf dst, kr_buf src, size_t len);                    /* :362 */
int kr_mul(kr_ctx* ctx, kr_buf out, size_t out_off, kr_buf a, size_t a_off, kr_buf b,    /* :370-379 */
           size_t b_off, size_t len);
int kr_conv_prefill(kr_ctx* ctx, kr_buf out, kr_buf x, kr_buf kernel, size_t rows,        /* :388 */
                    size_t dim, size_t k);
int kr_conv_decode(kr_ctx* ctx, kr_buf out, kr_buf x, kr_buf kernel, kr_buf state,        /* :397 */
                   size_t dim, size_t k);
int kr_silu_mul(kr_ctx* ctx, kr_buf gate, kr_buf up, size_t len);                        /* :400 */
int kr_logits(kr_ctx* ctx, kr_buf x, kr_buf y);                                          /* :403 */

/* ---- the same kernels on an unbound matrix (no model needed) */
/* Cpu::project arithmetic (cpu.rs:304-371 with the int8 path): rows of x
 * [rows, in_dim] -> y [rows, out_dim]. */
int kr_matmul(kr_ctx* ctx, kr_mat w, kr_buf x, kr_buf y, size_t rows);
/* Cpu::logits arithmetic (cpu.rs:501-514) with `w` as the classifier. */
int kr_classify(kr_ctx* ctx, kr_mat w, kr_buf x, kr_buf y);

/* kr_matmul for callers that cannot allocate device memory (code being
 * captured into a HIP graph, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same arguments and the same
 * results as kr_matmul, but the quantized activations go to a fixed device
 * array of kr_matmul_noalloc_max_elems() elements (4 Mi: 4.75 MiB with the
 * scales) that each device holds from the first kr_open on it until the
 * process ends, so the call itself makes no allocating call. Fails with
 * KR_ERR_INVALID when rows * in_dim exceeds that limit. All calls on one
 * device share the array: calls that overlap in time on one device (two
 * contexts' streams, or two threads) race; calls on one context's stream
 * are ordered and safe. */
int kr_matmul_noalloc(kr_ctx* ctx, kr_mat w, kr_buf x, kr_buf y, size_t rows);
size_t kr_matmul_noalloc_max_elems(void);

/* The two halves of kr_matmul, as Cpu::project runs them (quantize_rows,
 * cpu.rs:143-158, then the batched kernel): quantize rows of x into the
 * context's activation workspace, then run the projection kernel on it. */
int kr_quantize_rows(kr_ctx* ctx, kr_buf x, size_t rows, size_t width);
int kr_matmul_quantized(kr_ctx* ctx, kr_mat w, kr_buf y, size_t rows);
/* The fused launch behind project_qkv / project_gate_up (mod.rs:326-337):
 * n (1..3) matrices with the same in_dim and storage, one kernel launch over
 * all their rows, on the quantized workspace rows; y[i] gets w[i]'s output. */
int kr_matmul_quantized_set(kr_ctx* ctx, const kr_mat* w, const kr_buf* y, int n, size_t rows);

/* The chain-split form of kr_matmul for a Q8_0 matrix with in_dim % 128 == 0,
 * the one the prefill driver runs for few rows. No counterpart in the
 * reference: it computes the same four partial sums per output as
 * Matrix::matmul's Q8_0 kernel (dot.rs:34-45) -- t[j] over the blocks
 * b = j mod 4, in block order -- each on its own workgroups, and leaves them
 * as four planes y[j][rows][out_dim] (y holds 4 * rows * out_dim floats);
 * ((y[0] + y[1]) + y[2]) + y[3] is kr_matmul's output bit for bit. x: rows
 * of width in_dim, quantized into the workspace in chain-major block order;
 * KR_NO_BUF reuses the workspace as the previous kr_matmul_split left it.
 * The matrix's chain-major copy (out_dim * in_dim * 1.125 bytes) is made on
 * first use and kept until the matrix is freed. */
int kr_matmul_split(kr_ctx* ctx, kr_mat w, kr_buf x, kr_buf y, size_t rows);

/* A bare streaming read of len floats of src from `offset` (both multiples
 * of 4): the practical ceiling of a read-dominated kernel of that size, for
 * benchmarks. No counterpart in the reference. */
int kr_stream_read(kr_ctx* ctx, kr_buf src, size_t offset, size_t len);
/* The same read with its shape chosen: chunks_per_lane 16-byte loads per
 * lane per round (1, 2, 4, 8), on `workgroups` workgroups of 256 threads
 * (0: as many as one round each needs; fewer loop over the data). Used to
 * sweep for the best bare read of each launch size. kr_stream_read is
 * chunks_per_lane 2, workgroups 0. */
int kr_stream_read_shape(kr_ctx* ctx, kr_buf src, size_t offset, size_t len, int chunks_per_lane,
                         size_t workgroups);

/* An int8 MFMA throughput probe for benchmarks (no counterpart in the
 * reference): `workgroups` x 4 waves, each keeping four independent int8 MFMAs
 * in flight for `iters` rounds (kind 0: v_mfma_i32_32x32x32_i8, kind 1:
 * v_mfma_i32_16x16x32_i8); *ops gets the int8 operations issued. Time it with
 * kr_timer_start / kr_timer_stop to measure the chip's dense int8 rate.
 * workgroups x iters is capped at 2^32 (about half a second of MFMA work). */
int kr_mfma_rate(kr_ctx* ctx, int kind, size_t workgroups, size_t iters, double* ops);

/* Launch capture: the ops issued between kr_capture_begin and
 * kr_capture_end are recorded into one HIP graph instead of running (so
 * their inputs must stay alive and unchanged); kr_replay launches that
 * graph `times` times on the context's stream. No counterpart in the
 * reference; it lets a benchmark issue a fixed op sequence the way the
 * model driver's captured decode step does. */
int kr_capture_begin(kr_ctx* ctx);
int kr_capture_end(kr_ctx* ctx);
int kr_replay(kr_ctx* ctx, size_t times);

/* Stream-ordered timing: events recorded on the context's stream. */
int kr_timer_start(kr_ctx* ctx);
int kr_timer_stop(kr_ctx* ctx, float* ms); /* waits for the stop event */

/* ---- parity probes for the bit-exact int8 stages */
/* Activation quantization of `rows` rows of `width` (cpu.rs:143-158 /
 * quant.rs:856-874): quants [rows*width], scales [rows*width/32], f16 bits. */
int kr_dbg_quantize(kr_ctx* ctx, kr_buf x, size_t rows, size_t width, int8_t* quants,
                    float* scales, uint16_t* scales_f16);
/* Per-block exact i32 dot products of `w`'s rows with the quantized rows of
 * x: out [rows][out_dim][in_dim/32], through the same dot code as kr_matmul. */
int kr_dbg_block_dots(kr_ctx* ctx, kr_mat w, kr_buf x, size_t rows, int32_t* out);

/* One v_mfma_f32_32x32x1_2b_f32 per group on host operands: a, b [groups][64]
 * (lane l: block l / 32, row / column l % 32), acc and out [groups][32][64]
 * (register v of lane l; registers 16 blk .. +15 hold block blk's 32 x 32
 * outputs, element (8 (j / 4) + 4 (l / 32) + j % 4, l % 32) in register
 * 16 blk + j). The prefill GEMM's scale products and the prefill attention's
 * chains rely on every output being fmaf(a, b, acc); a test checks it with
 * this. groups <= 4096. No counterpart in the reference. */
int kr_dbg_mfma_f32(kr_ctx* ctx, const float* a, const float* b, const float* acc, float* out, size_t groups);

/* The serial f32 sum of each of `count` vectors of n non-negative values
 * (values [count][n], n <= 2048): s = +0, s += v[i] in order, as the
 * reference's RMS and softmax sums (cpu.rs:635-641, cpu.rs:575-630), by
 * the kernels' parallel exact form over `waves` waves (1, 2, 4 or 16) and by the
 * one-wave chain. out [count][5]: the parallel form's sum bits, 1 if it
 * applied (else the kernels use the chain), the chain's sum bits, and the
 * shader clocks each took. No counterpart in the reference. */
int kr_dbg_serial_sum(kr_ctx* ctx, const float* values, size_t n, size_t count, int waves, uint32_t* out);

/* A device matrix as stored: row-major int8 quants [out_dim][in_dim] and the
 * block scales [out_dim][in_dim/32] (f32 for Q8_0, f16 bits for Q8_0x4) --
 * so a host checker can rebuild the reference's Matrix from the very bytes a
 * kernel reads (e.g. the device-generated synthetic weights). */
int kr_matrix_read(kr_ctx* ctx, kr_mat m, int8_t* quants, size_t quants_bytes, void* scales,
                   size_t scales_bytes); /* the byte sizes must be the matrix's exactly */
/* out_dim, in_dim and storage (KR_STORAGE_*) of a device matrix. */
int kr_matrix_shape(kr_ctx* ctx, kr_mat m, size_t* out_dim, size_t* in_dim, int* storage);

/* ---- key/value cache access, for benchmarks that start from a filled cache */
/* which: 0 keys, 1 values; element offset into [n_layers, seq_len, kv_dim]. */
int kr_kv_upload(kr_ctx* ctx, int which, size_t offset, const float* data, size_t len);
int kr_kv_read(kr_ctx* ctx, int which, size_t offset, float* out, size_t len);
int kr_kv_synthetic(kr_ctx* ctx, size_t slots, uint64_t seed); /* N(0,1) into slots [0,slots) */

/* ---- device-side helpers for on-device greedy decoding */
/* argmax with the reference's tie rule (generate.rs:70-77) of buf[0..len),
 * written as an integer into tokens[index] (a device token ring). */
int kr_argmax(kr_ctx* ctx, kr_buf x, size_t len, size_t index);
/* Host copy of the device token ring. */
int kr_read_tokens(kr_ctx* ctx, size_t* out, size_t n);

int kr_synchronize(kr_ctx* ctx);

#ifdef __cplusplus
}
#endif

#endif /* KERNRT_HIP_H */

// gfx950 kernels of the KernRT HIP backend.
//
// Exactness contract: every kernel reproduces the f32 rounding sequence of
// the reference KernRT CPU backend on x86 (src/backends/cpu.rs and the ops it
// calls), so results are bit-identical to it, not merely close. Integer work
// (quantized dots) is order-free; floating-point reductions keep the
// reference's order, and only order-free work (per-element products,
// per-block integer dots, maxima) is spread across lanes. Build with
// -ffp-contract=off; fma appears only where the reference writes `mul_add`.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device.hpp"
#include "kernels.hpp"
#include "numerics.hpp"

namespace kr {

static constexpr int kStorageQ8_0 = 2;

typedef int v4i __attribute__((ext_vector_type(4)));


// Serial f32 chains, software-pipelined: operands are fetched in batches of
// kPipe elements, the next batch's loads issued before the current batch's
// dependent operations, so each step waits only on the previous one, never
// on a memory read. The last batch may be partial: its loads are clamped to
// the last element (n is uniform across the lanes that call these) and only
// its first n % kPipe steps are applied. The accumulation order is exactly
// left to right.
static constexpr int kPipe = 16;

template <typename T, typename Load, typename Op>
__device__ __forceinline__ float seq_chain(float acc, uint32_t n, Load&& load, Op&& op) {
    if (n == 0) return acc;
    const uint32_t nbt = (n + kPipe - 1) / kPipe;
    auto fetch = [&](T(&r)[kPipe], uint32_t b) {  // a whole batch: contiguous loads
#pragma unroll
        for (int j = 0; j < kPipe; j++) r[j] = load(b * kPipe + j);
    };
    auto fetch_last = [&](T(&r)[kPipe], uint32_t b) {
#pragma unroll
        for (int j = 0; j < kPipe; j++) r[j] = load(min(b * kPipe + j, n - 1));
    };
    auto apply = [&](const T(&r)[kPipe]) {
#pragma unroll
        for (int j = 0; j < kPipe; j++) acc = op(acc, r[j]);
    };
    T cur[kPipe];
    if (nbt == 1)
        fetch_last(cur, 0);
    else
        fetch(cur, 0);
    for (uint32_t b = 1; b + 1 < nbt; b++) {
        T nxt[kPipe];
        fetch(nxt, b);
        apply(cur);
#pragma unroll
        for (int j = 0; j < kPipe; j++) cur[j] = nxt[j];
    }
    if (nbt > 1) {
        T nxt[kPipe];
        fetch_last(nxt, nbt - 1);
        apply(cur);
#pragma unroll
        for (int j = 0; j < kPipe; j++) cur[j] = nxt[j];
    }
    const uint32_t last = n - (nbt - 1) * kPipe;  // 1..kPipe
#pragma unroll
    for (int j = 0; j < kPipe; j++)
        if ((uint32_t)j < last) acc = op(acc, cur[j]);
    return acc;
}

// ((0 + a[0]) + a[1]) + ... + a[n-1]
__device__ __forceinline__ float seq_sum(const float* __restrict__ a, uint32_t n) {
    return seq_chain<float>(0.0f, n, [&](uint32_t i) { return a[i]; }, [](float s, float v) { return s + v; });
}

// acc += p[j] * t[j * stride] for j in order (mul then add, unfused)
__device__ __forceinline__ float seq_dot(float acc, const float* __restrict__ p, const float* __restrict__ t,
                                         uint32_t stride, uint32_t n) {
    return seq_chain<float>(acc, n, [&](uint32_t i) { return p[i] * t[i * stride]; },
                            [](float s, float v) { return s + v; });
}

// slot = fma(e[b].x, e[b].y, slot) for b in order (quant.rs:287)
__device__ __forceinline__ float seq_fma(const float2* __restrict__ e, uint32_t n) {
    return seq_chain<float2>(0.0f, n, [&](uint32_t i) { return e[i]; },
                             [](float s, float2 v) { return __builtin_fmaf(v.x, v.y, s); });
}

// Two blocks' exact sums from one lane pair: for chunks u0 and u1 the even
// lane holds the dots of the first 16 bytes of each block (d0, d1), the odd
// lane those of the second 16 bytes. One swap gives the even lane block u0
// and the odd lane block u1, so each lane finishes one block's epilogue
// instead of both lanes of the pair repeating it.
__device__ __forceinline__ int pair_blocks(int d0, int d1, bool even) {
    const int recv = __builtin_amdgcn_mov_dpp(even ? d1 : d0, 0xB1, 0xf, 0xf, false);
    return (even ? d0 : d1) + recv;
}
__device__ __forceinline__ int dot16(const v4i& w, const v4i& x) {
    int acc = 0;
    acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
    acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
    acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
    return __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
}



// ---------------------------------------------------------------------------
// Activation quantization (quant.rs:856-874 per row, cpu.rs:143-158 batched).
// One 32-lane half-wave per Q8 block: lanes load one element each, the block
// amax is a 32-lane max reduction (max is order-free), then every lane
// rounds its own element.
__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ x, size_t total_blocks,
                                                  uint32_t nb, uint32_t k, size_t x_stride,
                                                  int8_t* __restrict__ q, float* __restrict__ s,
                                                  uint16_t* __restrict__ h, uint32_t cm) {
    size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
    size_t blk = gid >> 5;
    int lane = threadIdx.x & 31;
    bool valid = blk < total_blocks;
    size_t row = valid ? blk / nb : 0, b = valid ? blk % nb : 0;
    float v = valid ? x[row * x_stride + b * 32 + lane] : 0.0f;
    float m = fmaxf(0.0f, fabsf(v));  // fold(0.0, max(|v|)), NaN-ignoring
    m = group_max32(m);
    float d = div_rn(m, 127.0f);
    float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
    if (valid) {
        const size_t pb = row * nb + (cm ? cm_block((uint32_t)b, nb) : (uint32_t)b);  // cm: chain-major order
        q[pb * 32 + lane] = q8_round(v * inv);
        if (lane == 0) {
            s[pb] = d;
            h[pb] = f16_bits(d);
        }
    }
}

hipError_t launch_quantize(hipStream_t st, const float* x, size_t rows, size_t k, size_t x_stride,
                           int8_t* q, float* s, uint16_t* h, bool chain_major) {
    size_t nb = k / 32, total = rows * nb;
    if (total == 0) return hipSuccess;
    if (chain_major && nb % 4 != 0) return hipErrorInvalidValue;
    size_t threads = total * 32;
    dim3 grid((unsigned)((threads + 255) / 256));
    hipLaunchKernelGGL(k_quantize, grid, dim3(256), 0, st, x, total, (uint32_t)nb, (uint32_t)k, x_stride,
                       q, s, h, chain_major ? 1u : 0u);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Quantized GEMV (M <= 4 activation rows).
//
// A workgroup owns a tile of R consecutive weight rows, i.e. R*K contiguous
// bytes of the row-major int8 matrix. Thread t takes the 16-byte chunks
// t, t+256, t+512, ... of the tile, so every wave load is 1 KiB, fully
// coalesced. All of a thread's loads are issued before any is used -- its
// weight chunks, the matching activation chunks and the two scales of the
// blocks it finishes -- and none sits behind a branch, so a tile costs one
// memory round trip. A lane pair holds the two 16-byte halves of a 32-byte
// Q8 block: each lane does four v_dot4_i32_i8 on its half, so the per-block
// i32 is exact. Chunks go in pairs (u0, u1): one lane swap hands the even
// lane the whole of block u0 and the odd lane the whole of block u1, and
// each lane turns its block into the reference's epilogue operand and parks
// it in LDS (half the epilogue instructions of a pair in which both lanes
// finish each block); after one barrier the f32 chains run
// in the reference order: one lane per output for the FMA chain
// (quant.rs:276-288), four lanes per output for the four partial sums
// (dot.rs:35-44), which are joined as ((t0 + t1) + t2) + t3.
//
// One launch may cover up to three matrices with the same K (q/k/v, or
// gate/up): the grid is the concatenation of their tile ranges.
// LDS layout of the epilogue operands of one output (one weight row for one
// activation row). Four partial sums: residue j of the blocks at
// [j*q4p, j*q4p + count_j), q4p = ceil(nb/4) + 1 (odd, so the four lanes
// of an output and neighbouring outputs hit different banks). FMA chain:
// (isum, scale) pairs, nb + 1 of them per output.
__host__ __device__ inline uint32_t gemv_q4p(uint32_t nb) { return (nb + 3) / 4 + 1; }
__host__ __device__ inline uint32_t gemv_out_floats(int sem, uint32_t nb) {
    return sem == SEM_FMA_CHAIN ? 2 * (nb + 1) : 4 * gemv_q4p(nb);
}

// Serial f32 sum of n LDS values in order: each run of 16 loads is issued
// at once and then summed, one LDS round trip per 16 values.
__device__ __forceinline__ float lds_sum(const float* e, uint32_t n) {
    float t = 0.0f;
    uint32_t i = 0;
    for (; i + 16 <= n; i += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = e[i + j];
#pragma unroll
        for (int j = 0; j < 16; j++) t += v[j];
    }
    if (i < n) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = i + j < n ? e[i + j] : 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (i + j < n) t += v[j];
    }
    return t;
}

// Workgroup barrier that waits only for this wave's LDS operations
// (lgkmcnt(0)), not for its outstanding global loads or stores: for phases
// that communicate through LDS while other global traffic is in flight. The
// asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    __asm__ __volatile__("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt(63) expcnt(7) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __asm__ __volatile__("" ::: "memory");
}

// Serial f32 sum s += e[i], i = 0..n-1 in order, over 16-byte aligned LDS:
// 32 values per batch (8 x b128), the next batch's loads issued before the
// current batch's adds, so the LDS round trip overlaps the dependent adds
// and the chain runs at the add latency. Every batch load is unconditional
// (the last one re-reads a valid batch), which keeps the compiler's wait
// before each batch at lgkmcnt(8) instead of 0.
__device__ __forceinline__ float chain_sum(const float* __restrict__ e, uint32_t n, float s = 0.0f) {
    const uint32_t nb = n / 32;
    float4 A[8], B[8];
    auto ld = [&](float4(&r)[8], uint32_t b) {
#pragma unroll
        for (int u = 0; u < 8; u++) r[u] = *(const float4*)(e + 32 * b + 4 * u);
    };
    auto add = [&](const float4(&r)[8]) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            s += r[u].x;
            s += r[u].y;
            s += r[u].z;
            s += r[u].w;
        }
    };
    // one wait per batch: lgkmcnt(8), the batch before the one just issued
    // (LDS reads of a wave complete in order); a wait per value would cost
    // the chain about 0.8 clocks per add
    constexpr int kWaitPrev = 0xC07F | (8 << 8);
    uint32_t b = 0;
    if (nb > 0) ld(A, 0);
    for (; b + 2 <= nb; b += 2) {
        ld(B, b + 1);
        __builtin_amdgcn_s_waitcnt(kWaitPrev);
        __builtin_amdgcn_sched_barrier(0);
        add(A);
        ld(A, b + 2 < nb ? b + 2 : b);
        __builtin_amdgcn_s_waitcnt(kWaitPrev);
        __builtin_amdgcn_sched_barrier(0);
        add(B);
    }
    if (b < nb) add(A);
    for (uint32_t i = 32 * nb; i < n; i++) s += e[i];
    return s;
}

// Serial f32 sum s += e[i], i = 0..n-1 in order, run by one whole wave
// (all 64 lanes call it; every lane gets the sum): lane L first loads
// e[64 L .. 64 L + 63] into registers (all lanes at once, so the LDS round
// trip is paid once), then the chain passes from lane to lane: every lane
// adds its values to its running sum in order -- only lane L's is the
// chain -- and a DPP wave_shr:1 move hands lane L's sum to lane L + 1 as its
// start. Register-fed dependent adds run at ~4.5 clocks each against ~8-9
// for an LDS-fed one-lane chain; a hand-off costs ~25 clocks, once per 64
// values. Past n the values are zeros (e[n .. round4(n)) is cleared first,
// later ones are not loaded), and adding +0.0 leaves a sum of non-negative
// terms unchanged, so every lane adds all 64 of its values and the code has
// one path. e is 16-byte aligned LDS, writable up to round4(n), holding
// values >= 0 (squares, exponentials); n <= 64 VPL (VPL values per lane:
// fewer registers for a few more hand-offs).
template <int VPL = 64>
__device__ __forceinline__ float wave_chain_sum(float* __restrict__ e, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63, base = lane * VPL, n4 = (n + 3) & ~3u;
    if (lane < n4 - n) e[n + lane] = 0.0f;  // a wave's LDS accesses complete in order
    float v[VPL];
#pragma unroll
    for (int u = 0; u < VPL / 4; u++) {
        const float4 f = base + 4 * u < n4 ? *(const float4*)(e + base + 4 * u) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        v[4 * u] = f.x, v[4 * u + 1] = f.y, v[4 * u + 2] = f.z, v[4 * u + 3] = f.w;
    }
    const uint32_t runs = (n + VPL - 1) / VPL;
    float acc = 0.0f;
    for (uint32_t L = 0; L < runs; L++) {
#pragma unroll
        for (int k = 0; k < VPL; k++) acc += v[k];
        if (L + 1 < runs)  // wave_shr:1 -- lane L + 1 continues from lane L
            acc = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x138, 0xf, 0xf, false));
    }
    return runs ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), runs - 1)) : 0.0f;
}

// Two serial sums in one pass, one per half-wave: lanes 0..31 run e0's chain
// as wave_chain_sum<64> does and lanes 32..63 run e1's (n0, n1 <= 1024). The
// wave-wide shift also hands lane 31's running sum to lane 32 after every
// run; that sum only ever holds values of e0 past position 1024 (lanes 16 and
// up, at most 16 runs), which are zeros, so lane 32 starts from +0 as lane 0
// does. A chain that is done before the other one moves on through lanes
// whose values are zeros, and x + (+0) = x for these non-negative sums, so
// both end in the last lane of their half that the runs reach.
__device__ __forceinline__ float2 wave_chain_sum2(float* __restrict__ e0, uint32_t n0, float* __restrict__ e1,
                                                  uint32_t n1) {
    const uint32_t lane = threadIdx.x & 63, hl = lane & 31;
    float* e = lane < 32 ? e0 : e1;
    const uint32_t n = lane < 32 ? n0 : n1, n4 = (n + 3) & ~3u, base = hl * 64;
    if (hl < n4 - n) e[n + hl] = 0.0f;  // a wave's LDS accesses complete in order
    float v[64];
#pragma unroll
    for (int u = 0; u < 16; u++) {
        const float4 f = base + 4 * u < n4 ? *(const float4*)(e + base + 4 * u) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        v[4 * u] = f.x, v[4 * u + 1] = f.y, v[4 * u + 2] = f.z, v[4 * u + 3] = f.w;
    }
    const uint32_t r0 = (n0 + 63) / 64, r1 = (n1 + 63) / 64, runs = r0 > r1 ? r0 : r1;
    float acc = 0.0f;
    for (uint32_t L = 0; L < runs; L++) {
#pragma unroll
        for (int k = 0; k < 64; k++) acc += v[k];
        if (L + 1 < runs)  // wave_shr:1
            acc = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x138, 0xf, 0xf, false));
    }
    if (runs == 0) return make_float2(0.0f, 0.0f);
    return make_float2(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), runs - 1)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 32 + runs - 1)));
}

// ---- exact serial sums, evaluated in parallel --------------------------------
//
// The reference's serial sums of non-negative terms (the RMS sum of squares,
// the softmax sum of exponentials) are s_{k+1} = fl(s_k + a_k) from s_0 = +0.
// wave_exact_sum gives the same bits without a chain of n dependent adds:
//
//   While s stays in one binade [2^e, 2^(e+1)) it is a multiple of that
//   binade's ulp g = 2^(e-23), and so is each rounded result; then
//   fl(s + a) = s + g * rne(a / g) unless a / g is exactly halfway between two
//   integers (a tie, whose rounding depends on the last bit of s). So inside
//   a binade the sum is s plus an exact integer sum of per-term roundings,
//   which can be added in any order.
//
// The terms are split into segments of predicted binade: an approximate
// prefix sum (f32, any order) predicts the binade of each partial sum s_{k+1};
// a term whose predicted binade differs from its predecessor's (the sum
// crosses a power of two there), or that is a tie in its binade's grid, is a
// "special" term. Every other term contributes r_k = rne(a_k / g) to an
// integer scan. Then one short chain over the specials in order does, per
// special k: s += g * (sum of r over the segment before k) -- exact -- and
// s = fl(s + a_k) on the vector unit, the reference's own rounding. Each
// segment is verified exactly: its start is in the predicted binade and its
// end below the binade's top (the sums are monotone, so every partial sum in
// between is in the binade too, and every r_k used the right grid). If any
// check fails, if a term is not finite, if there are more than 63 specials
// or a term is too large for its grid, the function reports failure and the
// caller runs the serial chain (wave_chain_sum). Binade 1 is merged with the
// subnormals (the same ulp, 2^-149), so +0 starts in it.
//
// One wave holds the terms lane-major (lane L: terms L*VPL .. L*VPL+VPL-1):
// two passes of ~17 vector operations per term over 64 lanes, two scans, and
// a chain of ~10-20 specials read from their lanes, against n dependent adds
// for the serial chain.
// Inclusive wave scans (lane L gets the sum over lanes 0..L).
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}
__device__ __forceinline__ float wave_scan_f32(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xa, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xc, 0xf, false));
    return x;
}

// Binade bucket of a non-negative float: the biased exponent, with the
// subnormals and +0 in bucket 1 (the grid of bucket b is 2^(b - 150)).
__device__ __forceinline__ uint32_t xs_bucket(float p) { return max((uint32_t)__float_as_uint(p), 0x00800000u) >> 23; }

// LDS scratch of one exact sum: the specials' steps in order (up to 64 and
// the tail, then 8 no-op steps the chain may read past the last one), one
// dump slot per lane for the branch-free compaction, the waves' totals.
template <int W>
struct XsScratch {
    uint4 rec[72 + 64];
    float wtot[W];
    uint32_t wq[W], wc[W], wbad[W];
};

// e: 16-byte aligned LDS holding n <= 64 W VPL non-negative values, with
// e[n .. round4(n)) == +0; xs: scratch private to this sum. W == 1: one wave
// calls it (all 64 lanes); W > 1: every thread of the workgroup calls it
// (three workgroup barriers) and waves 0..W-1 share the terms. The result is
// valid in wave 0: true and the sum in `out`, or false, after which wave 0
// runs the chain.
template <int VPL, int W>
__device__ __forceinline__ bool block_exact_sum(const float* __restrict__ e, uint32_t n, XsScratch<W>* __restrict__ xs,
                                                float& out) {
    static_assert(VPL % 4 == 0 && VPL <= 32 && (W & (W - 1)) == 0 && W <= 16, "values per lane, waves");
    const uint32_t lane = threadIdx.x & 63, wave = W == 1 ? 0u : threadIdx.x >> 6;
    const bool active = W == 1 || wave < (uint32_t)W;
    const uint32_t n4 = (n + 3) & ~3u, k0 = (wave * 64 + lane) * VPL;
    auto sync = [&]() {
        if constexpr (W > 1) __syncthreads();
        else __builtin_amdgcn_wave_barrier();
    };
    float v[VPL];
#pragma unroll
    for (int u = 0; u < VPL / 4; u++) {
        const uint32_t k = k0 + 4 * u;
        const bool in = active && k < n4;
        const float4 f = *(const float4*)(e + (in ? k : 0));  // no branch; terms past n are zeros
        v[4 * u] = in ? f.x : 0.0f, v[4 * u + 1] = in ? f.y : 0.0f;
        v[4 * u + 2] = in ? f.z : 0.0f, v[4 * u + 3] = in ? f.w : 0.0f;
    }
    // pass 1: the lane's total and the approximate prefix before it
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++) acc += v[j];
    const float incl = wave_scan_f32(acc);
    float wbase = 0.0f, tot;
    if constexpr (W > 1) {
        if (lane == 63 && active) xs->wtot[wave] = incl;
        __syncthreads();
        tot = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            if ((uint32_t)w == wave) wbase = tot;
            tot += xs->wtot[w];
        }
    } else {
        tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), 63));
    }
    const float base = wbase + (incl - acc);
    // the bucket before each lane's first term: the previous lane's last, as
    // pass 2 computes it; +0 (bucket 1) before the first term; none before a
    // wave's first term past wave 0 (which makes that term special), unless
    // the wave holds only zeros past n (its constant bucket: no specials)
    uint32_t ep = xs_bucket(base + acc);
    const int ep0 = wave == 0 ? 1 : wave * 64 * VPL < n ? -1 : (int)xs_bucket(wbase);  // a wave of zeros: none
    ep = (uint32_t)__builtin_amdgcn_update_dpp(ep0, (int)ep, 0x138, 0xf, 0xf, false);  // wave_shr:1
    // pass 2: buckets, specials, per-term roundings and their lane prefix; a
    // rounding is capped at 2^24 (a term that large fails its segment check)
    uint32_t qv[VPL], bv[VPL / 4];
    uint32_t q = 0, spec = 0;
    float a2 = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++) {
        a2 += v[j];
        const uint32_t b = xs_bucket(base + a2);
        const float x = __builtin_amdgcn_ldexpf(v[j], 150 - (int)b);
        const float r = __builtin_rintf(x);
        const bool sp = b != ep || fabsf(x - r) == 0.5f;
        q += sp ? 0u : (uint32_t)fminf(r, 16777216.0f);
        qv[j] = q;
        if ((j & 3) == 0) bv[j >> 2] = 0;
        bv[j >> 2] |= b << (8 * (j & 3));
        spec |= (uint32_t)sp << j;
        ep = b;
    }
    // a term not finite or a sum that overflows; a lane below 2^26 keeps a
    // wave's integer scan below 2^32, a total below 2^31 keeps every prefix
    // exact (a valid sum has at most 64 segments of less than 2^23 each)
    const bool bad = !(tot < __builtin_huge_valf()) || q >= (1u << 26);
    const uint32_t cnt = __builtin_popcount(spec);
    const uint32_t rin = wave_scan_u32(q), cin = wave_scan_u32(cnt);
    uint32_t qoff = 0, coff = 0, nspec, qtot;
    bool anybad = __builtin_amdgcn_ballot_w64(bad) != 0;
    if constexpr (W > 1) {
        if (lane == 63 && active) xs->wq[wave] = rin, xs->wc[wave] = cin, xs->wbad[wave] = anybad ? 1u : 0u;
        __syncthreads();
        uint64_t q64 = 0;
        uint32_t nb = 0;
        nspec = 0;
#pragma unroll
        for (int w = 0; w < W; w++) {
            if ((uint32_t)w == wave) qoff = (uint32_t)q64, coff = nspec;
            q64 += xs->wq[w], nspec += xs->wc[w], nb |= xs->wbad[w];
        }
        anybad = nb != 0 || q64 >= (1ull << 31);
        qtot = (uint32_t)q64;
    } else {
        nspec = __builtin_amdgcn_readlane(cin, 63), qtot = __builtin_amdgcn_readlane(rin, 63);
        anybad |= qtot >= (1u << 31);
    }
    if (anybad || nspec > 63) return false;  // uniform over the workgroup
    // the specials at their rank in term order: term index, integer prefix,
    // the term's bucket (that of the segment after it), the term; the other
    // terms go to the lane's dump slot (no branches)
    if (active) {
        uint32_t rank = coff + cin - cnt;
        const uint32_t qb = qoff + rin - q;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const uint32_t sp = (spec >> j) & 1u;
            xs->rec[sp ? rank : 72 + lane] =
                make_uint4(k0 + j, qb + qv[j], (bv[j >> 2] >> (8 * (j & 3))) & 0xffu, __float_as_uint(v[j]));
            rank += sp;
        }
    }
    sync();
    if (W > 1 && wave != 0) return false;
    // step t (lane t): the segment before special t (from the previous
    // special, or from +0 in bucket 1) and the special; step nspec: the tail
    // segment, no term; later steps: no-ops. Step = (d, a, lo, top): s += d
    // is the segment's exact sum, lo <= s and s + d <= top (the float below
    // the bucket's end; the largest float for a no-op, so that an overflow
    // fails) verify its bucket, then s = fl(s + a).
    constexpr float kTopAll = 3.40282347e38f;
    {
        const uint4 cur = lane < nspec ? xs->rec[lane] : make_uint4(64u * W * VPL, qtot, 0u, 0u);
        const uint4 prv = lane > 0 && lane <= nspec ? xs->rec[lane - 1] : make_uint4(0xffffffffu, 0u, 1u, 0u);
        const uint32_t t = cur.y - prv.y, b = prv.z;
        const bool ne = lane <= nspec && cur.x - prv.x > 1u;
        float4 st;
        st.x = ne ? __builtin_amdgcn_ldexpf((float)t, (int)b - 150) : 0.0f;
        st.y = lane < nspec ? __uint_as_float(cur.w) : 0.0f;
        st.z = ne && b > 1u ? __uint_as_float(b << 23) : 0.0f;
        st.w = ne ? __uint_as_float(((b + 1u) << 23) - 1u) : kTopAll;
        __builtin_amdgcn_wave_barrier();
        ((float4*)xs->rec)[lane] = st;
        if (lane < 8) ((float4*)xs->rec)[64 + lane] = make_float4(0.0f, 0.0f, 0.0f, kTopAll);
    }
    __builtin_amdgcn_wave_barrier();
    // the chain, eight steps per LDS wait; the checks fold into
    // m = min(s - lo, top - (s + d)) >= 0 (a difference of floats is negative
    // exactly when the first is smaller)
    float s = 0.0f, m = 1.0f;
    for (uint32_t i0 = 0; i0 <= nspec; i0 += 8) {
        float4 r8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) r8[u] = ((const float4*)xs->rec)[i0 + u];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float lo = s - r8[u].z;
            s += r8[u].x;
            m = fminf(m, fminf(lo, r8[u].w - s));
            s += r8[u].y;
        }
    }
    out = s;
    return m >= 0.0f;
}

// The serial sum by the fast path where it applies, else by the chain (CVPL
// values per lane) on wave 0. W > 1: every thread of the workgroup calls it;
// the sum is valid in wave 0.
template <int VPL, int W, int CVPL = 64>
__device__ __forceinline__ float block_serial_sum(float* __restrict__ e, uint32_t n, XsScratch<W>* __restrict__ xs) {
    float s = 0.0f;
    if (n <= 64u * W * VPL) {
        const bool ok = block_exact_sum<VPL, W>(e, n, xs, s);
        if (W > 1 && (threadIdx.x >> 6) != 0) return 0.0f;
        if (ok) return s;
    } else if (W > 1 && (threadIdx.x >> 6) != 0) {
        return 0.0f;
    }
    return n <= 64 * CVPL ? wave_chain_sum<CVPL>(e, n) : chain_sum(e, n);
}

// The RMS sum of squares (rms_norm_row, cpu.rs:635-641) in a workgroup of
// four or more waves, shared by waves 0..3: sq (LDS) holds the dim squares
// with sq[dim .. round4(dim)) == +0. Every thread calls it; the sum is valid
// in wave 0.
__device__ __forceinline__ float rms_sum4(float* __restrict__ sq, uint32_t dim) {
    __shared__ XsScratch<4> xs;
    if (dim <= 1024) return block_serial_sum<4, 4>(sq, dim, &xs);
    if (dim <= 2048) return block_serial_sum<8, 4>(sq, dim, &xs);
    return block_serial_sum<16, 4>(sq, dim, &xs);
}

// Lane k (0..3) of each quad, to every lane of the quad (DPP quad_perm).
template <int K>
__device__ __forceinline__ float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), K * 0x55, 0xf, 0xf, false));
}


template <int SEM, int M, int CPT>
__global__ __launch_bounds__(256) void k_gemv(MatSet ms, QuantAct x, uint32_t K, uint32_t R, uint32_t step_rows,
                                              uint32_t step_cols, int32_t* __restrict__ dbg) {
    extern __shared__ __align__(16) float res[];
    const int mi = blockIdx.x < ms.tile_end[0] ? 0 : (blockIdx.x < ms.tile_end[1] ? 1 : 2);
    const uint32_t tile = blockIdx.x - (mi == 0 ? 0 : ms.tile_end[mi - 1]);
    const int8_t* __restrict__ W = ms.q[mi];
    const void* __restrict__ WS = ms.s[mi];
    const uint32_t N = ms.n[mi];
    const uint32_t nb = K >> 5, kc = K >> 4;  // blocks and 16-byte chunks per row
    const uint32_t row0 = tile * R;
    const uint32_t rows = min(R, N - row0);
    const uint32_t C = rows * kc;  // chunks in this tile
    const uint32_t tid = threadIdx.x;
    constexpr bool WF16 = SEM != SEM_FOUR_PARTIALS_F32;
    constexpr bool XF16 = SEM == SEM_FMA_CHAIN;
    const int8_t* wt = W + (size_t)row0 * K;

    // chunk tid + 256u sits at (row, col) of the tile; 256 chunks further is
    // (step_rows, step_cols) further, with carry
    uint32_t row = tid / kc, col = tid - (tid / kc) * kc;
    // chunks 2v (even lane) and 2v + 1 (odd lane) are the blocks this lane
    // finishes; only their scales are loaded
    const bool even = (tid & 1) == 0;
    v4i wv[CPT], xv[CPT][M];
    uint32_t wsb[CPT / 2], xsb[CPT / 2][M], rowu[CPT / 2], blku[CPT / 2];
#pragma unroll
    for (int u = 0; u < CPT; u++) {
        const bool in = tid + 256 * u < C;
        const uint32_t rr = in ? row : rows - 1, cc = in ? col : kc - 1;  // clamped: no branch
        wv[u] = __builtin_nontemporal_load((const v4i*)(wt + (size_t)rr * K + cc * 16));
#pragma unroll
        for (int m = 0; m < M; m++) xv[u][m] = *(const v4i*)(x.q + (size_t)m * K + cc * 16);
        if ((u & 1) == 0) rowu[u / 2] = rr, blku[u / 2] = cc >> 1;
        else if (!even) rowu[u / 2] = rr, blku[u / 2] = cc >> 1;
        col += step_cols;
        row += step_rows;
        if (col >= kc) col -= kc, row += 1;
    }
#pragma unroll
    for (int v = 0; v < CPT / 2; v++) {
        const uint32_t b = blku[v];
        wsb[v] = scale_bits(WF16, WS, (size_t)(row0 + rowu[v]) * nb + b);
#pragma unroll
        for (int m = 0; m < M; m++) xsb[v][m] = XF16 ? (uint32_t)x.h[m * nb + b] : f2u(x.s[m * nb + b]);
    }

    const uint32_t per = gemv_out_floats(SEM, nb), q4p = gemv_q4p(nb);
    // LDS slots for the stores of lanes that own no block, one per lane: a
    // store of many lanes to one address is serialised like a bank conflict
    const uint32_t dummy = M * rows * per + 2 * (tid & 63);
#pragma unroll
    for (int v = 0; v < CPT / 2; v++) {
        const bool valid = tid + 256 * (even ? 2 * v : 2 * v + 1) < C;
        const uint32_t r = rowu[v], b = blku[v];
        const float ws = scale_value(WF16, wsb[v]);
#pragma unroll
        for (int m = 0; m < M; m++) {
            const int isum = pair_blocks(dot16(wv[2 * v], xv[2 * v][m]), dot16(wv[2 * v + 1], xv[2 * v + 1][m]), even);
            // every lane forms the operand and stores it (a lane whose chunk
            // is past the tile to a dummy slot): with no branch around the
            // use, the scale loads stay at the top of the kernel
            float v0, v1 = 0.0f;
            if (SEM == SEM_FMA_CHAIN) {
                // quant.rs: slot = (isum as f32).mul_add(f16w(ws) * f16w(xs), slot)
                v0 = (float)isum;
                v1 = ws * f16w((uint16_t)xsb[v][m]);
            } else {
                // dot.rs: t[b & 3] += (sa * sb) * (isum as f32)
                v0 = (ws * u2f(xsb[v][m])) * (float)isum;
            }
            const bool own = valid;
            if (dbg && own) dbg[((size_t)m * N + row0 + r) * nb + b] = isum;
            const uint32_t base = (m * rows + r) * per;
            if (SEM == SEM_FMA_CHAIN) {
                float2* o = (float2*)(res + (own ? base + 2 * b : dummy));
                *o = make_float2(v0, v1);
            } else {
                res[own ? base + (b & 3) * q4p + (b >> 2) : dummy] = v0;
            }
        }
    }
    __syncthreads();

    float* Y = ms.y[mi];
    const uint32_t ld = ms.ld[mi];
    const uint32_t outs = M * rows;
    if (SEM == SEM_FMA_CHAIN) {
        for (uint32_t o = tid; o < outs; o += 256) {
            const uint32_t m = o / rows, r = o - m * rows;
            Y[(size_t)m * ld + row0 + r] = seq_fma((const float2*)(res + (size_t)o * per), nb);
        }
    } else {
        // lanes 4o .. 4o+3 run the four chains of output o
        for (uint32_t base = 0; base < 4 * outs; base += 256) {
            const uint32_t i = base + tid, o = i >> 2, j = i & 3;
            float t = 0.0f;
            if (o < outs && j < nb) t = lds_sum(res + (size_t)o * per + j * q4p, (nb - j + 3) / 4);
            const float t0 = quad_bcast<0>(t), t1 = quad_bcast<1>(t), t2 = quad_bcast<2>(t), t3 = quad_bcast<3>(t);
            if (o < outs && j == 0) {
                const uint32_t m = o / rows, r = o - m * rows;
                Y[(size_t)m * ld + row0 + r] = ((t0 + t1) + t2) + t3;
            }
        }
    }
}

// Rows per workgroup tile: about 8 KiB of weights, two 16-byte chunks per
// thread (a sweep over R at the 360M and 1.7B shapes: 8 KiB tiles were the
// fastest or within 3% of it at every shape, from 960x960 to 16384x2048).
static size_t gemv_rows_per_tile(size_t n, size_t k) {
    size_t r = 8192 / k;
    if (r < 1) r = 1;
    if (r > n) r = n;
    if (r > 256) r = 256;
    return r;
}

template <int SEM, int M, int CPT>
static void gemv_go(hipStream_t st, const MatSet& ms, QuantAct x, uint32_t k, uint32_t R, uint32_t total,
                    size_t lds, int32_t* dbg) {
    const uint32_t kc = k / 16;
    hipLaunchKernelGGL((k_gemv<SEM, M, CPT>), dim3(total), dim3(256), lds, st, ms, x, k, R, 256 / kc, 256 % kc,
                       dbg);
}

template <int SEM, int M>
static hipError_t gemv_launch(hipStream_t st, MatSet ms, size_t k, QuantAct x, int32_t* dbg) {
    size_t n_max = 0;
    for (int i = 0; i < ms.count; i++) n_max = ms.n[i] > n_max ? ms.n[i] : n_max;
    const size_t R = gemv_rows_per_tile(n_max, k);
    uint32_t total = 0;
    for (int i = 0; i < 3; i++) {
        if (i < ms.count) total += (uint32_t)((ms.n[i] + R - 1) / R);
        ms.tile_end[i] = total;
    }
    const size_t lds = ((size_t)M * R * gemv_out_floats(SEM, (uint32_t)(k / 32)) + 128) * sizeof(float);
    const size_t chunks = R * (k / 16);
    const size_t cpt = (chunks + 255) / 256;
    if (cpt <= 2)
        gemv_go<SEM, M, 2>(st, ms, x, (uint32_t)k, (uint32_t)R, total, lds, dbg);
    else if (cpt <= 4)
        gemv_go<SEM, M, 4>(st, ms, x, (uint32_t)k, (uint32_t)R, total, lds, dbg);
    else if (cpt <= 8)
        gemv_go<SEM, M, 8>(st, ms, x, (uint32_t)k, (uint32_t)R, total, lds, dbg);
    else
        return hipErrorInvalidValue;  // k > 32768: rejected when the matrix is made
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode GEMV with the producer of its activation fused in front (M = 1).
//
// A decode step alternates a short serial producer (the residual add +
// RMSNorm + quantization, or the quantization of an f32 row) with a GEMV that
// must wait for it. Run as two launches, the GEMV's weight fetch cannot start
// until the producer ends. Here every workgroup issues the producer's loads
// (L2-resident, a few KiB), then its weight loads, and computes the producer
// while the weights are in flight: the serial RMS sum (dim dependent adds,
// the reference order) overlaps the HBM round trip instead of preceding it.
// The quantized row is built in LDS with the exact arithmetic of the
// standalone kernels (k_add_rms_quant, k_quantize), so the results are
// bit-identical to running those and then k_gemv. Workgroup 0 writes the
// updated residual row to a second buffer (the other workgroups still read
// the old one).
struct GemvPro {
    const float* a;  // PRO_NORM: residual row x; PRO_QUANT: the f32 row
    const float* b;  // PRO_NORM: the add into x (may be null)
    const float* w;  // PRO_NORM: norm weight
    float* x_out;    // PRO_NORM: x + add, written by workgroup 0 (may be null)
    float eps;
};
static constexpr int PRO_NORM = 1, PRO_QUANT = 3;

// The producer of k_gemv_pro / k_gemv_swiglu, after its inputs were loaded
// into registers (va: the residual row or the f32 row, vb: the add, vw: the
// norm weight): with PRO_NORM the residual add, the serial RMS sum (in its
// exact parallel form; rms_norm_row, cpu.rs:635-641) and out = w * (scale *
// x) (cpu.rs:643);
// then Q8Vec::quantize_into (quant.rs:864-873) of the row into LDS (xq, and
// the scale values xsb: f16-rounded for the FMA-chain format, else f32), a block per 8
// threads. Every thread of the workgroup calls this; the row is spread over
// threads 0..255 (VPT float4 each), further threads only join the barriers.
template <int SEM, int PRO, int VPT, int CVPL = 64, int NW = 4>
__device__ __forceinline__ void gemv_produce(const GemvPro& pro, uint32_t K, float4 (&va)[VPT], const float4 (&vb)[VPT],
                                             const float4 (&vw)[VPT], int8_t* xq, uint32_t* xsb, float* scratch,
                                             float* s_scale_p) {
    constexpr bool XF16 = SEM == SEM_FMA_CHAIN;
    const uint32_t tid = threadIdx.x, n4 = K >> 2;
    float4 o[VPT];
    if constexpr (PRO == PRO_NORM) {
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const uint32_t f = tid + 256 * u;
            if (f < n4) {
                float4 v = va[u];
                if (pro.b) v = make_float4(v.x + vb[u].x, v.y + vb[u].y, v.z + vb[u].z, v.w + vb[u].w);
                va[u] = v;
                if (blockIdx.x == 0 && pro.x_out) ((float4*)pro.x_out)[f] = v;
                ((float4*)scratch)[f] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
            }
        }
        __syncthreads();
        // rms_norm_row (cpu.rs:635-641): the serial sum of the squares in its
        // exact parallel form over the workgroup's NW waves (the chain on
        // wave 0 where that does not apply); every thread takes part in its
        // barriers
        __shared__ XsScratch<NW> xs;
        float ss = 0.0f;
        if constexpr (NW >= 16) {
            ss = block_serial_sum<4, NW, CVPL>(scratch, K, &xs);
        } else {
            ss = K <= 1024 ? block_serial_sum<4, NW, CVPL>(scratch, K, &xs) : block_serial_sum<8, NW, CVPL>(scratch, K, &xs);
        }
        if (tid < 64) {
            ss = div_rn(ss, (float)K);
            ss += pro.eps;
            if (tid == 0) *s_scale_p = div_rn(1.0f, sqrt_rn(ss));
        }
        __syncthreads();
        const float scale = *s_scale_p;
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            const float4 v = va[u], wq = vw[u];
            o[u] = make_float4(wq.x * (scale * v.x), wq.y * (scale * v.y), wq.z * (scale * v.z), wq.w * (scale * v.w));
        }
    } else {
        static_assert(PRO == PRO_QUANT, "producer kind");
#pragma unroll
        for (int u = 0; u < VPT; u++) o[u] = va[u];
    }
    // Q8Vec::quantize_into (quant.rs:864-873) into LDS; a block is 8 threads
#pragma unroll
    for (int u = 0; u < VPT; u++) {
        const uint32_t f = tid + 256 * u;
        if (f < n4) {  // K % 32 == 0: the 8 threads of a block are all in range or all out
            const float4 v = o[u];
            float m = fmaxf(fmaxf(fmaxf(fmaxf(0.0f, fabsf(v.x)), fabsf(v.y)), fabsf(v.z)), fabsf(v.w));
            m = group_max8(m);
            const float d = div_rn(m, 127.0f);
            const float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
            char4 qq;
            qq.x = q8_round(v.x * inv);
            qq.y = q8_round(v.y * inv);
            qq.z = q8_round(v.z * inv);
            qq.w = q8_round(v.w * inv);
            ((char4*)xq)[f] = qq;
            // the block scale as the epilogue uses it: f16-rounded and widened
            // (quant.rs:276-288) for the FMA-chain format, else the f32 scale
            if ((f & 7) == 0) xsb[f / 8] = f2u(XF16 ? f16w(f16_bits(d)) : d);
        }
    }
    __syncthreads();
}

template <int SEM, int PRO, int VPT>
__global__ __launch_bounds__(256) void k_gemv_pro(MatSet ms, GemvPro pro, uint32_t K, uint32_t R,
                                                  uint32_t step_rows, uint32_t step_cols) {
    constexpr int CPT = 2;  // rows per tile keep R * K <= 8 KiB
    // LDS: x quants [K] | x scale bits [nb] | scratch: squares [K], then the epilogue operands
    extern __shared__ __align__(16) float sm[];
    __shared__ float s_scale;
    const int mi = blockIdx.x < ms.tile_end[0] ? 0 : (blockIdx.x < ms.tile_end[1] ? 1 : 2);
    const uint32_t tile = blockIdx.x - (mi == 0 ? 0 : ms.tile_end[mi - 1]);
    const int8_t* __restrict__ W = ms.q[mi];
    const void* __restrict__ WS = ms.s[mi];
    const uint32_t nb = K >> 5, kc = K >> 4, n4 = K >> 2;
    const uint32_t row0 = tile * R;
    const uint32_t rows = min(R, ms.n[mi] - row0);
    const uint32_t C = rows * kc;
    const uint32_t tid = threadIdx.x;
    constexpr bool WF16 = SEM != SEM_FOUR_PARTIALS_F32;
    int8_t* xq = (int8_t*)sm;
    uint32_t* xsb = (uint32_t*)(sm + n4);
    float* scratch = sm + ((n4 + nb + 3) & ~3u);

    // 1. the producer's inputs first, so waiting for them never waits for the weights
    float4 va[VPT], vb[VPT], vw[VPT];
#pragma unroll
    for (int u = 0; u < VPT; u++) {
        const uint32_t f = tid + 256 * u;
        if (f < n4) {
            va[u] = ((const float4*)pro.a)[f];
            vb[u] = pro.b ? ((const float4*)pro.b)[f] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (PRO == PRO_NORM) vw[u] = ((const float4*)pro.w)[f];
        }
    }
    // 2. the weight tile, as k_gemv loads it
    const int8_t* wt = W + (size_t)row0 * K;
    uint32_t row = tid / kc, col = tid - (tid / kc) * kc;
    static_assert(CPT == 2, "one block per lane: chunk 0 on even lanes, chunk 1 on odd lanes");
    const bool even = (tid & 1) == 0;
    v4i wv[CPT];
    uint32_t rowu[CPT], colu[CPT];
#pragma unroll
    for (int u = 0; u < CPT; u++) {
        const bool in = tid + 256 * u < C;
        const uint32_t rr = in ? row : rows - 1, cc = in ? col : kc - 1;
        rowu[u] = rr, colu[u] = cc;
        wv[u] = __builtin_nontemporal_load((const v4i*)(wt + (size_t)rr * K + cc * 16));
        col += step_cols;
        row += step_rows;
        if (col >= kc) col -= kc, row += 1;
    }
    const uint32_t r_own = even ? rowu[0] : rowu[1], b_own = (even ? colu[0] : colu[1]) >> 1;
    const uint32_t wsb = scale_bits(WF16, WS, (size_t)(row0 + r_own) * nb + b_own);

    // 3. the producer, while the weights are in flight
    gemv_produce<SEM, PRO, VPT>(pro, K, va, vb, vw, xq, xsb, scratch, &s_scale);

    // 4. block dots against the LDS row, then the epilogue of k_gemv
    const uint32_t per = gemv_out_floats(SEM, nb), q4p = gemv_q4p(nb);
    float* res = scratch;
    const uint32_t dummy = rows * per + 2 * (tid & 63);  // a slot per lane, as in k_gemv
    {
        const bool own = tid + 256 * (even ? 0 : 1) < C;
        const uint32_t r = r_own, b = b_own;
        const float ws = scale_value(WF16, wsb);
        const float xs = u2f(xsb[b]);
        const v4i xv0 = *(const v4i*)(xq + colu[0] * 16), xv1 = *(const v4i*)(xq + colu[1] * 16);
        const int isum = pair_blocks(dot16(wv[0], xv0), dot16(wv[1], xv1), even);
        const uint32_t base = r * per;
        if (SEM == SEM_FMA_CHAIN) {
            float2* op = (float2*)(res + (own ? base + 2 * b : dummy));
            *op = make_float2((float)isum, ws * xs);
        } else {
            res[own ? base + (b & 3) * q4p + (b >> 2) : dummy] = (ws * xs) * (float)isum;
        }
    }
    __syncthreads();
    float* Y = ms.y[mi];
    if (SEM == SEM_FMA_CHAIN) {
        for (uint32_t oi = tid; oi < rows; oi += 256) Y[row0 + oi] = seq_fma((const float2*)(res + (size_t)oi * per), nb);
    } else {
        for (uint32_t base = 0; base < 4 * rows; base += 256) {
            const uint32_t i = base + tid, oi = i >> 2, j = i & 3;
            float t = 0.0f;
            if (oi < rows && j < nb) t = lds_sum(res + (size_t)oi * per + j * q4p, (nb - j + 3) / 4);
            const float t0 = quad_bcast<0>(t), t1 = quad_bcast<1>(t), t2 = quad_bcast<2>(t), t3 = quad_bcast<3>(t);
            if (oi < rows && j == 0) Y[row0 + oi] = ((t0 + t1) + t2) + t3;
        }
    }
}

template <int SEM, int PRO>
static hipError_t gemv_pro_go(hipStream_t st, MatSet ms, size_t k, const GemvPro& pro) {
    size_t n_max = 0;
    for (int i = 0; i < ms.count; i++) n_max = ms.n[i] > n_max ? ms.n[i] : n_max;
    const size_t R = gemv_rows_per_tile(n_max, k);
    if (R * (k / 16) > 512) return hipErrorInvalidValue;
    uint32_t total = 0;
    for (int i = 0; i < 3; i++) {
        if (i < ms.count) total += (uint32_t)((ms.n[i] + R - 1) / R);
        ms.tile_end[i] = total;
    }
    const size_t nb = k / 32, head = (k / 4 + nb + 3) & ~(size_t)3;
    const size_t ops = R * gemv_out_floats(SEM, (uint32_t)nb) + 128;
    const size_t lds = (head + (ops > k ? ops : k)) * sizeof(float);
    const size_t vpt = (k / 4 + 255) / 256;
    const uint32_t kc = (uint32_t)(k / 16);
#define KR_PRO_GO(V)                                                                                            \
    hipLaunchKernelGGL((k_gemv_pro<SEM, PRO, V>), dim3(total), dim3(256), lds, st, ms, pro, (uint32_t)k,         \
                       (uint32_t)R, 256 / kc, 256 % kc)
    if (vpt <= 1)
        KR_PRO_GO(1);
    else if (vpt <= 2)
        KR_PRO_GO(2);
    else if (vpt <= 4)
        KR_PRO_GO(4);
    else
        KR_PRO_GO(8);
#undef KR_PRO_GO
    return hipGetLastError();
}

hipError_t launch_project_pro(hipStream_t st, int sem, const DevMatrix* const* w, float* const* y, int count,
                              int pro_kind, const float* a, const float* b, const float* norm_w, float* x_out,
                              float eps) {
    if (count < 1 || count > 3 || (pro_kind != PRO_NORM && pro_kind != PRO_QUANT)) return hipErrorInvalidValue;
    const size_t k = w[0]->k;
    if (k % 32 != 0 || k > 8192) return hipErrorInvalidValue;
    MatSet ms{};
    ms.count = count;
    for (int i = 0; i < count; i++) {
        if (w[i]->k != k || w[i]->storage != w[0]->storage) return hipErrorInvalidValue;
        ms.q[i] = w[i]->q;
        ms.s[i] = w[i]->s;
        ms.y[i] = y[i];
        ms.n[i] = (uint32_t)w[i]->n;
        ms.ld[i] = (uint32_t)w[i]->n;
    }
    GemvPro pro{a, b, norm_w, x_out, eps};
#define KR_PRO_SEM(P)                                                                          \
    switch (sem) {                                                                             \
        case SEM_FMA_CHAIN: return gemv_pro_go<SEM_FMA_CHAIN, P>(st, ms, k, pro);              \
        case SEM_FOUR_PARTIALS_F32: return gemv_pro_go<SEM_FOUR_PARTIALS_F32, P>(st, ms, k, pro); \
        case SEM_FOUR_PARTIALS_F16: return gemv_pro_go<SEM_FOUR_PARTIALS_F16, P>(st, ms, k, pro); \
    }
    if (pro_kind == PRO_NORM) {
        KR_PRO_SEM(PRO_NORM)
    } else {
        KR_PRO_SEM(PRO_QUANT)
    }
#undef KR_PRO_SEM
    return hipErrorInvalidValue;
}

// Decode gate/up with the SwiGLU product and its quantization fused behind
// (M = 1, K <= 2048). Workgroup t computes rows 32 t .. 32 t + 31 of both the
// gate and the up matrix, with the residual add + RMSNorm + Q8 producer in
// front exactly as k_gemv_pro<PRO_NORM>; then one half-wave forms
// h = silu(gate) * up (cpu.rs:708-710, then cpu.rs:494-499) for those 32
// rows and quantizes them as Q8 block t of h (quant.rs:864-873) — the input
// of the down projection. The results are bit-identical to k_gemv_pro
// followed by k_silu_quant, with one launch fewer per layer. Tile row r < 32
// is gate row 32 t + r, r >= 32 up row 32 t + r - 32.
static constexpr uint32_t kSwigluMaxK = 2048;
static constexpr uint32_t kSwigluThreads = 1024;  // the producer runs on the first 256, VPT float4 each
template <int SEM, int CPT, int VPT>
__global__ __launch_bounds__(kSwigluThreads) void k_gemv_swiglu(MatSet ms, GemvPro pro, uint32_t K, uint32_t step_rows,
                                                     uint32_t step_cols, int8_t* __restrict__ hq,
                                                     float* __restrict__ hsc, uint16_t* __restrict__ hh,
                                                     float* __restrict__ hf) {
    constexpr uint32_t RT = 64;         // tile rows: 32 gate + 32 up
    extern __shared__ __align__(16) float sm[];  // x quants [K] | x scale bits [nb] | squares, then epilogue operands
    __shared__ float s_scale;
    __shared__ float s_out[RT];
    __shared__ uint64_t etab[32];
    constexpr uint32_t NT = kSwigluThreads;
    const uint32_t t = blockIdx.x;
    const uint32_t nb = K >> 5, kc = K >> 4, n4 = K >> 2, C = RT * kc;
    const uint32_t tid = threadIdx.x;
    constexpr bool WF16 = SEM != SEM_FOUR_PARTIALS_F32;
    int8_t* xq = (int8_t*)sm;
    uint32_t* xsb = (uint32_t*)(sm + n4);
    float* scratch = sm + ((n4 + nb + 3) & ~3u);
    const uint64_t etv = kExp2Tab[tid & 31];  // stored to LDS after every load is issued

    // 1. the producer's inputs first, so waiting for them never waits for the weights
    float4 va[VPT], vb[VPT], vw[VPT];
#pragma unroll
    for (int u = 0; u < VPT; u++) {
        const uint32_t f = tid + 256 * u;
        if (f < n4) {
            va[u] = ((const float4*)pro.a)[f];
            vb[u] = pro.b ? ((const float4*)pro.b)[f] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            vw[u] = ((const float4*)pro.w)[f];
        }
    }
    // 2. the weight tile: chunk tid + NT u is (tile row, 16-byte column). The
    // two matrices' bases are read once (uniform) and selected per chunk: an
    // argument array indexed per lane would be loaded from memory per lane.
    // chunk 2v (even lane) or 2v + 1 (odd lane) is the block a lane finishes
    static_assert(CPT % 2 == 0, "chunks pair up");
    const bool even = (tid & 1) == 0;
    v4i wv[CPT];
    uint32_t colu[CPT], wsb[CPT / 2], rowo[CPT / 2], blko[CPT / 2];
    {
        const int8_t* const wq0 = ms.q[0];
        const int8_t* const wq1 = ms.q[1];
        const void* const ws0 = ms.s[0];
        const void* const ws1 = ms.s[1];
        uint32_t row = tid / kc, col = tid - (tid / kc) * kc;
#pragma unroll
        for (int u = 0; u < CPT; u++) {
            const bool in = tid + NT * u < C;
            const uint32_t rr = in ? row : RT - 1, cc = in ? col : kc - 1;
            const bool up_row = rr >= 32;
            const uint32_t grow = 32 * t + (rr & 31);
            colu[u] = cc;
            wv[u] = __builtin_nontemporal_load((const v4i*)((up_row ? wq1 : wq0) + (size_t)grow * K + cc * 16));
            if ((u & 1) == 0) rowo[u / 2] = rr, blko[u / 2] = cc >> 1;
            else if (!even) rowo[u / 2] = rr, blko[u / 2] = cc >> 1;
            col += step_cols;
            row += step_rows;
            if (col >= kc) col -= kc, row += 1;
        }
#pragma unroll
        for (int v = 0; v < CPT / 2; v++) {
            const uint32_t rr = rowo[v];
            wsb[v] = scale_bits(WF16, rr >= 32 ? ws1 : ws0, (size_t)(32 * t + (rr & 31)) * nb + blko[v]);
        }
    }
    if (tid < 32) etab[tid] = etv;  // read after the producer's barriers
    // 3. the producer, while the weights are in flight
    // with eight chunks per thread in flight the chain holds 32 values a lane
    gemv_produce<SEM, PRO_NORM, VPT, CPT >= 8 ? 32 : 64, 4>(pro, K, va, vb, vw, xq, xsb, scratch, &s_scale);

    // 4. block dots against the LDS row, the epilogue operands to LDS
    const uint32_t per = gemv_out_floats(SEM, nb), q4p = gemv_q4p(nb);
    float* res = scratch;
    const uint32_t dummy = RT * per + 2 * (tid & 63);  // a slot per lane, as in k_gemv
#pragma unroll
    for (int v = 0; v < CPT / 2; v++) {
        const bool own = tid + NT * (even ? 2 * v : 2 * v + 1) < C;
        const uint32_t r = rowo[v], b = blko[v];
        const float ws = scale_value(WF16, wsb[v]);
        const float xs = u2f(xsb[b]);
        const v4i xv0 = *(const v4i*)(xq + colu[2 * v] * 16), xv1 = *(const v4i*)(xq + colu[2 * v + 1] * 16);
        const int isum = pair_blocks(dot16(wv[2 * v], xv0), dot16(wv[2 * v + 1], xv1), even);
        const uint32_t base = r * per;
        if (SEM == SEM_FMA_CHAIN) {
            float2* op = (float2*)(res + (own ? base + 2 * b : dummy));
            *op = make_float2((float)isum, ws * xs);
        } else {
            res[own ? base + (b & 3) * q4p + (b >> 2) : dummy] = (ws * xs) * (float)isum;
        }
    }
    __syncthreads();
    // 5. each row's chain in reference order (quant.rs:276-288 or dot.rs:35-44)
    if (SEM == SEM_FMA_CHAIN) {
        if (tid < RT) s_out[tid] = seq_fma((const float2*)(res + (size_t)tid * per), nb);
    } else {
        const uint32_t oi = tid >> 2, j = tid & 3;  // threads 0..255 = 64 rows x 4 partial sums
        float v = 0.0f;
        if (oi < RT && j < nb) v = lds_sum(res + (size_t)oi * per + j * q4p, (nb - j + 3) / 4);
        const float t0 = quad_bcast<0>(v), t1 = quad_bcast<1>(v), t2 = quad_bcast<2>(v), t3 = quad_bcast<3>(v);
        if (oi < RT && j == 0) s_out[oi] = ((t0 + t1) + t2) + t3;
    }
    __syncthreads();
    // 6. h = silu(gate) * up and its Q8 block, on the first half-wave
    if (tid < 32) {
        const float g = s_out[tid], up = s_out[32 + tid];
        const float h = div_rn(g, 1.0f + glibc_expf(-g, etab)) * up;
        if (hf) hf[32 * t + tid] = h;
        quant_lane(h, true, hq + 32 * t + tid, hsc + t, hh + t);
    }
}

hipError_t launch_gate_up_swiglu(hipStream_t st, int sem, const DevMatrix& gate, const DevMatrix& up, const float* x,
                                 const float* add, const float* norm_w, float* x_out, float eps, int8_t* hq,
                                 float* hs, uint16_t* hh, float* hf) {
    const size_t k = gate.k, n = gate.n;
    if (!swiglu_fusable(gate, up)) return hipErrorInvalidValue;
    MatSet ms{};
    ms.count = 2;
    ms.q[0] = gate.q, ms.s[0] = gate.s, ms.n[0] = (uint32_t)n;
    ms.q[1] = up.q, ms.s[1] = up.s, ms.n[1] = (uint32_t)n;
    GemvPro pro{x, add, norm_w, x_out, eps};
    const size_t nb = k / 32, kc = k / 16, head = (k / 4 + nb + 3) & ~(size_t)3;
    const size_t ops = 64 * gemv_out_floats(sem, (uint32_t)nb) + 128;
    const size_t lds = (head + (ops > k ? ops : k)) * sizeof(float);
    const size_t cpt = (64 * kc + kSwigluThreads - 1) / kSwigluThreads;
    const dim3 grid((unsigned)(n / 32));
    const size_t vpt = (k / 4 + 255) / 256;
#define KR_SWIGLU(SEMV, CPTV, VPTV)                                                                                    \
    hipLaunchKernelGGL((k_gemv_swiglu<SEMV, CPTV, VPTV>), grid, dim3(kSwigluThreads), lds, st, ms, pro, (uint32_t)k, \
                       (uint32_t)(kSwigluThreads / kc), (uint32_t)(kSwigluThreads % kc), hq, hs, hh, hf)
#define KR_SWIGLU_CPT(SEMV)    \
    if (cpt <= 2)              \
        KR_SWIGLU(SEMV, 2, 1); \
    else if (cpt <= 4)         \
        KR_SWIGLU(SEMV, 4, 1); \
    else if (vpt <= 1)         \
        KR_SWIGLU(SEMV, 8, 1); \
    else                       \
        KR_SWIGLU(SEMV, 8, 2);
    switch (sem) {
        case SEM_FMA_CHAIN: KR_SWIGLU_CPT(SEM_FMA_CHAIN) break;
        case SEM_FOUR_PARTIALS_F32: KR_SWIGLU_CPT(SEM_FOUR_PARTIALS_F32) break;
        case SEM_FOUR_PARTIALS_F16: KR_SWIGLU_CPT(SEM_FOUR_PARTIALS_F16) break;
        default: return hipErrorInvalidValue;
    }
#undef KR_SWIGLU_CPT
#undef KR_SWIGLU
    return hipGetLastError();
}

bool swiglu_fusable(const DevMatrix& gate, const DevMatrix& up) {
    return gate.k == up.k && gate.n == up.n && gate.storage == up.storage && gate.k % 32 == 0 &&
           gate.k >= 64 && gate.k <= kSwigluMaxK && gate.n % 32 == 0 && gate.n > 0;
}

// ---------------------------------------------------------------------------
// Quantized GEMM on int8 MFMA (prefill and batched rows, M >= kGemmMinRows).
// The four-partial Q8_0 GEMM (dot.rs:35-44) is k_gemm_q8 in gemm.hip; this
// file holds the Q8_0x4 FMA chain (quant.rs:276-288, k_gemm_chain).
//
// v_mfma_i32_32x32x32_i8 multiplies a 32x32 int8 tile of activations by a
// 32x32 int8 tile of weights over K = 32, exactly one Q8 block, so each
// instruction yields the exact i32 block dots of a 32x32 output tile. Every
// block's dots go straight into the reference's f32 epilogue, so each output
// keeps the per-row path's rounding sequence.
//
// Operand layout: lane l feeds row l % 32 of the activation tile and column
// l % 32 of the weight tile with bytes 16*(l/32) .. +16 of the block; both
// operands use the same byte map, so the integer sum covers the block once.
// Accumulator v of lane l is output (row 8*(v/4) + 4*(l/32) + v%4, col l%32).
//
// The chain is serial, so each wave owns its own 32x32 tile over all of K;
// the workgroup tile is 32x128 and the 4 waves share the activation chunk.
// Operands are staged through LDS in chunks of KC = 4 blocks: every row's
// KC*32 bytes are read with coalesced 16-byte loads (whole cache lines),
// several chunks ahead in registers, and written to a double-buffered LDS
// tile whose rows are padded by 16 bytes so that the fragment reads of 32
// consecutive rows spread over all banks. One barrier per chunk.
//
// Workgroups are numbered XCD-aware: the row tiles that share a column tile
// of weights run on one XCD and share its L2.
typedef int v16i __attribute__((ext_vector_type(16)));
static constexpr size_t kGemmMinRows = 8;
// chunks each thread keeps in flight in registers (even: LDS buffer parity)
static constexpr int kGemmStages = 4;

// Workgroup ids are dispatched round-robin over the 8 XCDs; map them so that
// consecutive logical tiles run on one XCD.
__device__ __forceinline__ uint32_t xcd_tile(uint32_t id, uint32_t count) {
    const uint32_t per = count >> 3, rem = count & 7, xcd = id & 7, k = id >> 3;
    return xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
}

// One column tile of a matrix in the set; tile_end counts column tiles of
// width `cols`.
struct GemmPos {
    int mi;
    uint32_t m0, n0;
};
__device__ __forceinline__ GemmPos gemm_pos(const MatSet& ms, uint32_t mtiles, uint32_t cols) {
    const uint32_t L = xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t mt = L % mtiles, nt = L / mtiles;
    const int mi = nt < ms.tile_end[0] ? 0 : (nt < ms.tile_end[1] ? 1 : 2);
    const uint32_t tile = nt - (mi == 0 ? 0 : ms.tile_end[mi - 1]);
    return GemmPos{mi, mt * 32, tile * cols};
}

// The 16 activation scales of accumulator rows 8g + 4*half + (0..3).
__device__ __forceinline__ void gemm_row_scales(float (&xs)[16], const float* col) {
    const float4* q = (const float4*)col;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float4 f = q[2 * g];
        xs[4 * g] = f.x, xs[4 * g + 1] = f.y, xs[4 * g + 2] = f.z, xs[4 * g + 3] = f.w;
    }
}

template <bool DBG>
__global__ __launch_bounds__(256, 2) void k_gemm_chain(MatSet ms, QuantAct x, uint32_t M, uint32_t K,
                                                       uint32_t mtiles, int32_t* __restrict__ dbg) {
    constexpr int KC = 4, ROW = KC * 32 + 16, NS = kGemmStages;
    __shared__ __align__(16) int8_t sA[2][32 * ROW];
    __shared__ __align__(16) int8_t sB[2][128 * ROW];
    __shared__ __align__(16) float sX[2][KC * 32];   // [block][row]
    __shared__ __align__(16) float sW[2][KC * 128];  // [block][col]
    const uint32_t nb = K >> 5, nchunks = (nb + KC - 1) / KC;
    const GemmPos p = gemm_pos(ms, mtiles, 128);
    const int8_t* __restrict__ W = ms.q[p.mi];
    const uint16_t* __restrict__ WS = (const uint16_t*)ms.s[p.mi];
    const uint32_t N = ms.n[p.mi];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: block checks branch on SGPRs
    const uint32_t r = lane & 31, half = lane >> 5;
    const uint32_t n = p.n0 + 32 * wave + r;       // this lane's output column
    const bool active = p.n0 + 32 * wave < N;       // uniform per wave

    // loader map: activation piece (row tid/8, 16-byte column tid%8), weight
    // pieces (rows tid/8 + 32i), activation scale (row (tid/4)%32, block
    // tid%4; the upper half of the workgroup repeats the lower), weight
    // scales (columns tid/4 + 64i, block tid%4).
    const uint32_t lr = tid >> 3, lc = (tid & 7) * 16, xr = (tid >> 2) & 31, wc = tid >> 2, sb = tid & 3;
    const int8_t* ga = x.q + (size_t)min(p.m0 + lr, M - 1) * K;
    const int8_t* gb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) gb[i] = W + (size_t)min(p.n0 + lr + 32 * i, N - 1) * K;
    const uint16_t* gx = x.h + (size_t)min(p.m0 + xr, M - 1) * nb;
    const size_t gw0 = (size_t)min(p.n0 + wc, N - 1) * nb, gw1 = (size_t)min(p.n0 + wc + 64, N - 1) * nb;

    struct Stage {
        v4i a, b[4];
        uint32_t xs, w0, w1;
    };
    auto gload = [&](Stage& st, uint32_t c) {
        c = c < nchunks ? c : nchunks - 1;
        const uint32_t col = min(c * KC * 32 + lc, K - 16);  // past the row end: a piece no block uses
        st.a = *(const v4i*)(ga + col);
#pragma unroll
        for (int i = 0; i < 4; i++) st.b[i] = *(const v4i*)(gb[i] + col);
        const uint32_t blk = min(c * KC + sb, nb - 1);
        st.xs = gx[blk];
        st.w0 = WS[gw0 + blk], st.w1 = WS[gw1 + blk];
    };
    auto lstore = [&](const Stage& st, int buf) {
        *(v4i*)(sA[buf] + lr * ROW + lc) = st.a;
#pragma unroll
        for (int i = 0; i < 4; i++) *(v4i*)(sB[buf] + (lr + 32 * i) * ROW + lc) = st.b[i];
        sX[buf][sb * 32 + xr] = f16w((uint16_t)st.xs);
        sW[buf][sb * 128 + wc] = f16w((uint16_t)st.w0);
        sW[buf][sb * 128 + wc + 64] = f16w((uint16_t)st.w1);
    };

    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    float slot[16];
#pragma unroll
    for (int v = 0; v < 16; v++) slot[v] = 0.0f;
    auto compute = [&](int buf, uint32_t c) {
        if (!active) return;
#pragma unroll
        for (int blk = 0; blk < KC; blk++) {
            const uint32_t b = c * KC + blk;
            if (b >= nb) break;
            const v4i a = *(const v4i*)(sA[buf] + r * ROW + blk * 32 + 16 * half);
            const v4i bq = *(const v4i*)(sB[buf] + (32 * wave + r) * ROW + blk * 32 + 16 * half);
            const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, zero, 0, 0, 0);
            const float w = sW[buf][blk * 128 + 32 * wave + r];
            float xs[16];
            gemm_row_scales(xs, sX[buf] + blk * 32 + 4 * half);
            if (DBG && n < N) {
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const uint32_t m = p.m0 + 8 * (v >> 2) + 4 * half + (v & 3);
                    if (m < M) dbg[((size_t)m * N + n) * nb + b] = d[v];
                }
            }
            // quant.rs: slot = (isum as f32).mul_add(f16w(ws) * f16w(xs), slot)
#pragma unroll
            for (int v = 0; v < 16; v++) slot[v] = __builtin_fmaf((float)d[v], w * xs[v], slot[v]);
        }
    };

    gemm_pipeline<NS, Stage>(nchunks, gload, lstore, compute);
    if (!active || n >= N) return;
    float* Y = ms.y[p.mi];
    const uint32_t ld = ms.ld[p.mi];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const uint32_t m = p.m0 + 8 * (v >> 2) + 4 * half + (v & 3);
        if (m < M) Y[(size_t)m * ld + n] = slot[v];
    }
}

template <int SEM>
static hipError_t gemm_launch(hipStream_t st, MatSet ms, size_t k, QuantAct x, size_t rows, int32_t* dbg) {
    if (SEM != SEM_FMA_CHAIN) return launch_gemm_q8(st, SEM, ms, k, x, rows, dbg);
    const uint32_t cols = 128;
    uint32_t total = 0;
    for (int i = 0; i < 3; i++) {
        if (i < ms.count) total += (uint32_t)((ms.n[i] + cols - 1) / cols);
        ms.tile_end[i] = total;
    }
    const uint32_t mtiles = (uint32_t)((rows + 31) / 32);
    dim3 grid(total * mtiles);
    const uint32_t m = (uint32_t)rows, kk = (uint32_t)k;
    if (dbg)
        hipLaunchKernelGGL(k_gemm_chain<true>, grid, dim3(256), 0, st, ms, x, m, kk, mtiles, dbg);
    else
        hipLaunchKernelGGL(k_gemm_chain<false>, grid, dim3(256), 0, st, ms, x, m, kk, mtiles, dbg);
    return hipGetLastError();
}

template <int SEM>
static hipError_t gemv_rows(hipStream_t st, const MatSet& ms, size_t k, QuantAct x, size_t rows, int32_t* dbg) {
    if (rows >= kGemmMinRows) return gemm_launch<SEM>(st, ms, k, x, rows, dbg);
    size_t nb = k / 32;
    size_t done = 0;
    while (done < rows) {
        size_t m = rows - done;
        QuantAct xm{x.q + done * k, x.s + done * nb, x.h + done * nb};
        MatSet mm = ms;
        for (int i = 0; i < ms.count; i++) mm.y[i] = ms.y[i] + done * ms.ld[i];
        int32_t* dm = dbg ? dbg + done * ms.n[0] * nb : nullptr;
        hipError_t e;
        if (m >= 4) {
            e = gemv_launch<SEM, 4>(st, mm, k, xm, dm);
            m = 4;
        } else if (m == 3) {
            e = gemv_launch<SEM, 3>(st, mm, k, xm, dm);
        } else if (m == 2) {
            e = gemv_launch<SEM, 2>(st, mm, k, xm, dm);
        } else {
            e = gemv_launch<SEM, 1>(st, mm, k, xm, dm);
        }
        if (e != hipSuccess) return e;
        done += m;
    }
    return hipSuccess;
}

hipError_t launch_project_set(hipStream_t st, int sem, const DevMatrix* const* w, float* const* y, int count,
                              QuantAct x, size_t rows, int32_t* dbg) {
    if (count < 1 || count > 3) return hipErrorInvalidValue;
    MatSet ms{};
    ms.count = count;
    for (int i = 0; i < count; i++) {
        if (w[i]->k != w[0]->k || w[i]->storage != w[0]->storage) return hipErrorInvalidValue;
        ms.q[i] = w[i]->q;
        ms.s[i] = w[i]->s;
        ms.y[i] = y[i];
        ms.n[i] = (uint32_t)w[i]->n;
        ms.ld[i] = (uint32_t)w[i]->n;
    }
    size_t k = w[0]->k;
    switch (sem) {
        case SEM_FMA_CHAIN: return gemv_rows<SEM_FMA_CHAIN>(st, ms, k, x, rows, dbg);
        case SEM_FOUR_PARTIALS_F32: return gemv_rows<SEM_FOUR_PARTIALS_F32>(st, ms, k, x, rows, dbg);
        case SEM_FOUR_PARTIALS_F16: return gemv_rows<SEM_FOUR_PARTIALS_F16>(st, ms, k, x, rows, dbg);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_project(hipStream_t st, int sem, const DevMatrix& w, QuantAct x, size_t rows, float* y,
                          size_t ldy, int32_t* dbg) {
    if (ldy != w.n) return hipErrorInvalidValue;
    const DevMatrix* ws[1] = {&w};
    float* ys[1] = {y};
    return launch_project_set(st, sem, ws, ys, 1, x, rows, dbg);
}

// ---------------------------------------------------------------------------
// RMSNorm (cpu.rs:633-644): ss is a left-to-right f32 sum of x*x; the squares
// are formed in parallel and summed by rms_sum4 with the same bits.
__global__ __launch_bounds__(256) void k_rms_norm(float* __restrict__ out, const float* __restrict__ x,
                                                  const float* __restrict__ w, uint32_t dim, float eps) {
    extern __shared__ __align__(16) float sq[];
    __shared__ float s_scale;
    const float* xr = x + (size_t)blockIdx.x * dim;
    float* orow = out + (size_t)blockIdx.x * dim;
    for (uint32_t i = threadIdx.x; i < dim; i += 256) {
        float v = xr[i];
        sq[i] = v * v;
    }
    if (threadIdx.x < ((dim + 3) & ~3u) - dim) sq[dim + threadIdx.x] = 0.0f;
    __syncthreads();
    float ss = rms_sum4(sq, dim);  // the sum in its exact parallel form
    if (threadIdx.x < 64) {
        ss = div_rn(ss, (float)dim);
        ss += eps;
        if (threadIdx.x == 0) s_scale = div_rn(1.0f, sqrt_rn(ss));
    }
    __syncthreads();
    float scale = s_scale;
    for (uint32_t i = threadIdx.x; i < dim; i += 256) orow[i] = w[i] * (scale * xr[i]);
}

hipError_t launch_rms_norm(hipStream_t st, float* out, const float* x, const float* w, size_t rows,
                           size_t dim, float eps) {
    if (rows == 0) return hipSuccess;
    size_t lds = ((dim + 3) & ~(size_t)3) * sizeof(float);
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)rows), dim3(256), lds, st, out, x, w, (uint32_t)dim, eps);
    return hipGetLastError();
}

// Per-head RMSNorm (cpu.rs:647-661), 16 lanes per (row, head): the squares
// of the head's values are formed in parallel into LDS, one lane runs the
// serial sum (the reference order), and the 16 lanes apply the scale to the
// values they hold in registers.
// Items 0 .. items1 - 1 are the heads of (v, width, w), the rest those of
// (v2, width2, w2): q and k of a layer in one launch.
__global__ __launch_bounds__(256) void k_qk_norm(float* __restrict__ v, uint32_t items, uint32_t width,
                                                 uint32_t head, const float* __restrict__ w, float eps,
                                                 uint32_t items1, float* __restrict__ v2, uint32_t width2,
                                                 const float* __restrict__ w2) {
    constexpr uint32_t MAXV = 16;  // values per lane: head <= 256
    extern __shared__ __align__(16) float sq[];  // [16 items][round4(head) + 4]
    __shared__ float s_scale[16];
    const uint32_t slot = threadIdx.x >> 4, l16 = threadIdx.x & 15;
    const uint32_t stride = ((head + 3) & ~3u) + 4;
    uint32_t item = blockIdx.x * 16 + slot;
    const bool live = item < items;
    if (item >= items1) item -= items1, v = v2, width = width2, w = w2;
    const uint32_t heads = width / head;
    float* hd = v + (size_t)(live ? item / heads : 0) * width + (size_t)(live ? item % heads : 0) * head;
    float* row = sq + slot * stride;
    float a[MAXV];
#pragma unroll
    for (uint32_t k = 0; k < MAXV; k++) {
        const uint32_t i = l16 + 16 * k;
        a[k] = live && i < head ? hd[i] : 0.0f;
        if (i < head) row[i] = a[k] * a[k];
    }
    __builtin_amdgcn_wave_barrier();  // a row's 16 lanes are in one wave: LDS order within the wave suffices
    if (l16 == 0) {  // rms of the head (cpu.rs:635-641 on one head)
        float ss = chain_sum(row, head);
        ss = div_rn(ss, (float)head);
        ss += eps;
        s_scale[slot] = div_rn(1.0f, sqrt_rn(ss));
    }
    __builtin_amdgcn_wave_barrier();
    const float scale = s_scale[slot];
#pragma unroll
    for (uint32_t k = 0; k < MAXV; k++) {
        const uint32_t i = l16 + 16 * k;
        if (live && i < head) hd[i] = w[i] * (scale * a[k]);
    }
}

hipError_t launch_qk_norm(hipStream_t st, float* v, size_t rows, size_t width, size_t head, const float* w,
                          float eps, float* v2, size_t width2, const float* w2) {
    const size_t n1 = rows * (width / head), n = n1 + (v2 ? rows * (width2 / head) : 0);
    if (n == 0) return hipSuccess;
    if (head > 256) return hipErrorInvalidValue;
    const size_t stride = ((head + 3) & ~(size_t)3) + 4;
    hipLaunchKernelGGL(k_qk_norm, dim3((unsigned)((n + 15) / 16)), dim3(256), 16 * stride * sizeof(float), st, v,
                       (uint32_t)n, (uint32_t)width, (uint32_t)head, w, eps, (uint32_t)n1, v2 ? v2 : v,
                       (uint32_t)(v2 ? width2 : width), v2 ? w2 : w);
    return hipGetLastError();
}

// RoPE (cpu.rs:664-705). (cos, sin) of every (position, frequency) come from
// a table the host builds with the same libm calls as the reference, so only
// the rotation itself runs here: two products and a difference/sum, unfused.
__global__ __launch_bounds__(256) void k_rope(float* __restrict__ q, float* __restrict__ k, uint32_t qw,
                                              uint32_t kvw, uint32_t rows, const uint32_t* __restrict__ pos,
                                              const float2* __restrict__ tab, uint32_t hs, int interleaved) {
    uint32_t half = hs / 2;
    uint32_t qpairs = interleaved ? qw / 2 : (qw / hs) * half;
    uint32_t kpairs = interleaved ? 0 : (kvw / hs) * half;
    uint32_t per_row = qpairs + kpairs;
    uint32_t id = blockIdx.x * 256 + threadIdx.x;
    if (id >= rows * per_row) return;
    uint32_t row = id / per_row, p = id % per_row;
    const float2* tr = tab + (size_t)pos[row] * half;
    if (interleaved) {
        uint32_t i = 2 * p;
        float2 cs = tr[(i % hs) / 2];
        float c = cs.x, s = cs.y;
        float* qv = q + (size_t)row * qw;
        float q0 = qv[i], q1 = qv[i + 1];
        qv[i] = q0 * c - q1 * s;
        qv[i + 1] = q0 * s + q1 * c;
        if (i < kvw) {
            float* kv = k + (size_t)row * kvw;
            float k0 = kv[i], k1 = kv[i + 1];
            kv[i] = k0 * c - k1 * s;
            kv[i + 1] = k0 * s + k1 * c;
        }
        return;
    }
    float* vec;
    uint32_t pp;
    if (p < qpairs) {
        vec = q + (size_t)row * qw;
        pp = p;
    } else {
        vec = k + (size_t)row * kvw;
        pp = p - qpairs;
    }
    uint32_t head = pp / half, i = pp % half;
    float2 cs = tr[i];
    float c = cs.x, s = cs.y;
    float* hd = vec + (size_t)head * hs;
    float lo = hd[i], hi = hd[i + half];
    hd[i] = lo * c - hi * s;
    hd[i + half] = lo * s + hi * c;
}

hipError_t launch_rope(hipStream_t st, float* q, float* k, size_t qw, size_t kvw, size_t rows,
                       const uint32_t* positions, const float2* table, size_t hs, int interleaved) {
    size_t half = hs / 2;
    size_t per_row = interleaved ? qw / 2 : (qw / hs) * half + (kvw / hs) * half;
    size_t n = rows * per_row;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, q, k, (uint32_t)qw,
                       (uint32_t)kvw, (uint32_t)rows, positions, table, (uint32_t)hs, interleaved);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_kv_write(float* __restrict__ kc, float* __restrict__ vc, size_t base,
                                                  uint32_t kv_dim, const uint32_t* __restrict__ slots,
                                                  const float* __restrict__ k, const float* __restrict__ v,
                                                  uint32_t rows) {
    uint32_t id = blockIdx.x * 256 + threadIdx.x;
    if (id >= rows * kv_dim) return;
    uint32_t row = id / kv_dim, e = id % kv_dim;
    size_t at = base + (size_t)slots[row] * kv_dim + e;
    kc[at] = k[id];
    vc[at] = v[id];
}

hipError_t launch_kv_write(hipStream_t st, float* kc, float* vc, size_t layer, size_t seq_len, size_t kv_dim,
                           const uint32_t* slots, const float* k, const float* v, size_t rows) {
    size_t n = rows * kv_dim;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_kv_write, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, kc, vc,
                       layer * seq_len * kv_dim, (uint32_t)kv_dim, slots, k, v, (uint32_t)rows);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Attention (cpu.rs:575-630), one workgroup per (query row, KV head): the
// kv_mul query heads that share a KV head are served together, so each K and
// V row is read once for all of them.
//  1. scores: one lane per cache row runs the reference's four-chain FMA dot
//     (dot.rs:350-366) against every query head of the group, times scale;
//  2. per-head max (order-free); exp via glibc's expf restated;
//  3. each head's softmax sum is left to right (one lane per head, side by
//     side in one wave), then every score / sum;
//  4. out[h][e] = sum_t p_t * v_t[e], one lane per (head, e), t in order.
//     V rows stream through two LDS tiles filled by all lanes; the first
//     tile's loads are issued together with the K loads of step 1.
// Scores live in LDS when they fit, otherwise in the caller's `att` rows.
static constexpr uint32_t kAttnThreads = 512;
static constexpr size_t kAttnLds = 150 * 1024;


__global__ __launch_bounds__(512) void k_attention(const float* __restrict__ q, float* __restrict__ out,
                                                   float* __restrict__ att, const float* __restrict__ kc,
                                                   const float* __restrict__ vc, size_t loff,
                                                   const DevWindow* __restrict__ windows, uint32_t n_heads,
                                                   uint32_t kv_mul, uint32_t hs, uint32_t kv_dim,
                                                   uint32_t seq_len, float scale, uint32_t G, uint32_t lds_scores,
                                                   uint32_t tile_rows, int8_t* __restrict__ qo,
                                                   float* __restrict__ so, uint16_t* __restrict__ ho) {
    // LDS: q [kv_mul][hs] | V tiles [2][tile_rows*hs] | scores [kv_mul][lds_scores]
    extern __shared__ float sm[];
    __shared__ float red[16][8];
    __shared__ float s_sum[8];
    __shared__ uint64_t etab[32];
    if (threadIdx.x < 32) etab[threadIdx.x] = kExp2Tab[threadIdx.x];  // read after the barriers below
    // this workgroup: query heads [h0, h0 + G), G | kv_mul, all on one KV head
    const uint32_t row = blockIdx.y, T = kAttnThreads;
    const DevWindow w = windows[row];
    const uint32_t n_shared = w.shared_end - w.shared_start;
    const uint32_t count = n_shared + w.slot - w.att_start + 1;
    const uint32_t width = n_heads * hs;
    const uint32_t h0 = blockIdx.x * G;
    const uint32_t kvo = (h0 / kv_mul) * hs;
    const uint32_t qn = G * hs;
    float* qs = sm;
    float* vt = sm + ((qn + 3) & ~3u);
    const uint32_t tile_f = tile_rows * hs;
    const bool sc_lds = count <= lds_scores;
    float* sc_base = sc_lds ? vt + 2 * tile_f : att + (size_t)row * n_heads * seq_len + (size_t)h0 * seq_len;
    const uint32_t sc_stride = sc_lds ? lds_scores : seq_len;  // per query head
    for (uint32_t e = threadIdx.x; e < qn; e += T) qs[e] = q[(size_t)row * width + (size_t)h0 * hs + e];

    // V tile loader: float4 f of the tile -> (row j, column col)
    const uint32_t tile_f4 = tile_f / 4;
    const uint32_t ntiles = (count + tile_rows - 1) / tile_rows;
    const float* vbase = vc + loff + kvo;
    constexpr int VPT = 8;  // float4 per lane per tile, enough for 16K floats
    float4 pre[VPT];
    auto load_tile = [&](uint32_t c) {
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            uint32_t f = threadIdx.x + T * u;
            pre[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (f < tile_f4) {
                uint32_t j = (4 * f) / hs, col = (4 * f) % hs, i = c * tile_rows + j;
                if (i < count) pre[u] = *(const float4*)(vbase + (size_t)win_slot(w, n_shared, i) * kv_dim + col);
            }
        }
    };
    auto store_tile = [&](uint32_t buf) {
#pragma unroll
        for (int u = 0; u < VPT; u++) {
            uint32_t f = threadIdx.x + T * u;
            if (f < tile_f4) *(float4*)(vt + buf * tile_f + 4 * f) = pre[u];
        }
    };
    load_tile(0);  // in flight while the scores are computed
    __syncthreads();

    // 1. scores
    float mx[8];
#pragma unroll
    for (int j = 0; j < 8; j++) mx[j] = -INFINITY;
    for (uint32_t i = threadIdx.x; i < count; i += T) {
        const float* kr = kc + loff + (size_t)win_slot(w, n_shared, i) * kv_dim + kvo;
        for (uint32_t j = 0; j < G; j++) {
            const float* qh = qs + j * hs;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            uint32_t e = 0;
#pragma unroll 8
            for (; e + 4 <= hs; e += 4) {
                float4 kk = *(const float4*)(kr + e);
                a0 = __builtin_fmaf(qh[e], kk.x, a0);
                a1 = __builtin_fmaf(qh[e + 1], kk.y, a1);
                a2 = __builtin_fmaf(qh[e + 2], kk.z, a2);
                a3 = __builtin_fmaf(qh[e + 3], kk.w, a3);
            }
            float d = (a0 + a1) + (a2 + a3);
            for (; e < hs; e++) d = __builtin_fmaf(qh[e], kr[e], d);
            float sv = d * scale;
            sc_base[j * sc_stride + i] = sv;
            if (j < 8) mx[j] = fmaxf(mx[j], sv);
        }
    }
    store_tile(0);
    for (uint32_t j = 0; j < G; j++) {
        float m = mx[j < 8 ? j : 0];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][j] = m;
    }
    __syncthreads();
    // 2. exp per (head, row) with the head's max
    for (uint32_t t = threadIdx.x; t < G * count; t += T) {
        uint32_t j = t / count, i = t % count;
        float m = red[0][j];
        for (uint32_t wv = 1; wv < T / 64; wv++) m = fmaxf(m, red[wv][j]);
        float* sc = sc_base + j * sc_stride;
        sc[i] = glibc_expf(sc[i] - m, etab);
    }
    __syncthreads();
    // 3. per-head sums, lanes 0..kv_mul-1 of wave 0 in lockstep
    if (threadIdx.x < G) s_sum[threadIdx.x] = seq_sum(sc_base + threadIdx.x * sc_stride, count);
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < G * count; t += T) {
        uint32_t j = t / count, i = t % count;
        float* sc = sc_base + j * sc_stride;
        sc[i] = div_rn(sc[i], s_sum[j]);
    }
    __syncthreads();

    // 4. weighted V sums: lane (j, e) for j < kv_mul, e < hs
    float acc[2] = {0.0f, 0.0f};  // lanes cover kv_mul*hs <= 2*T
    for (uint32_t c = 0; c < ntiles; c++) {
        if (c + 1 < ntiles) load_tile(c + 1);
        uint32_t rows = min(tile_rows, count - c * tile_rows);
#pragma unroll
        for (int r = 0; r < 2; r++) {
            uint32_t t = threadIdx.x + r * T;
            if (t < qn) {
                uint32_t j = t / hs, e = t % hs;
                acc[r] = seq_dot(acc[r], sc_base + j * sc_stride + c * tile_rows, vt + (c & 1) * tile_f + e, hs, rows);
            }
        }
        if (c + 1 < ntiles) store_tile((c + 1) & 1);
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
        uint32_t t = threadIdx.x + r * T;
        bool live = t < qn;
        size_t o = (size_t)row * width + (size_t)h0 * hs + t;
        if (live) out[o] = acc[r];
        // head outputs are whole Q8 blocks (hs % 32 == 0): quantize for o_proj
        if (qo && t < ((qn + 31) & ~31u)) quant_lane(acc[r], live, qo + o, so + o / 32, ho + o / 32);
    }
    // Leave the probabilities in `att` like the reference does.
    if (sc_lds) {
        for (uint32_t t = threadIdx.x; t < G * count; t += T) {
            uint32_t j = t / count, i = t % count;
            att[(size_t)row * n_heads * seq_len + (size_t)(h0 + j) * seq_len + i] = sc_base[j * sc_stride + i];
        }
    }
}

// ---------------------------------------------------------------------------
// Attention, latency-first form (the same arithmetic as k_attention).
//
// A decode step runs one query row against a few hundred cache rows, so the
// time is the critical path, not the work: the two serial chains per head
// (the softmax sum and the weighted V sum, each `count` dependent adds) plus
// the memory round trips before them. This form keeps the round trips few
// and off the chains:
//  * workgroup (head group, d-slice, row): the G query heads of one KV head
//    and DW of their HS output dims; the HS / DW slices of a group redo the
//    scores (cheap, parallel) so that each needs only count * DW floats of V;
//  * K rows are copied HBM -> LDS by the gfx950 LDS DMA
//    (global_load_lds_dwordx4), 16 bytes per lane, fully coalesced; the
//    float4 u of row r lands in slot u ^ (r % F) of its row (F float4 per
//    row), so when every lane then reads its own row the 16 lanes of a read
//    phase hit 16 different bank groups;
//  * one lane per cache row runs the reference dot (four FMA chains) for
//    every head of the group;
//  * the V slice is DMA'd into the same LDS by waves 1.. while wave 0 runs
//    the softmax sums, so its latency is hidden behind them;
//  * both chains read LDS in runs of 32-64 values per wait, at compile-time
//    offsets, which keeps a dependent add about every 8 cycles.
static constexpr uint32_t kAttnFastThreads = 512;

template <int G, int HS, int DW>
__global__ __launch_bounds__(512) void k_attention_fast(
    const float* __restrict__ q, float* __restrict__ out, float* __restrict__ att, const float* __restrict__ kc,
    const float* __restrict__ vc, size_t loff, const DevWindow* __restrict__ windows, uint32_t n_heads,
    uint32_t kv_mul, uint32_t kv_dim, uint32_t seq_len, float scale, uint32_t scs, uint32_t kcap, uint32_t vcap,
    int8_t* __restrict__ qo, float* __restrict__ so, uint16_t* __restrict__ ho) {
    constexpr uint32_t T = kAttnFastThreads, S = HS / DW, F = HS / 4, FV = DW / 4;
    // LDS: q [G][HS] | scores [G][scs] | work: K chunk [kcap][HS], later V [vcap][DW]
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[T / 64][G];
    __shared__ float s_sum[G];
    __shared__ uint64_t etab[32];  // the exp table, off the global memory path
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t row = blockIdx.y, hg = blockIdx.x / S, sidx = blockIdx.x % S;
    const DevWindow w = windows[row];
    const uint32_t n_shared = w.shared_end - w.shared_start;
    const uint32_t count = n_shared + w.slot - w.att_start + 1;  // <= scs: sized for the longest window
    const uint32_t width = n_heads * HS, d0 = sidx * DW;
    const uint32_t h0 = hg * G, kvo = (h0 / kv_mul) * HS;
    const float* __restrict__ qg = q + (size_t)row * width + (size_t)h0 * HS;
    float* sc = sm + G * HS;
    float* work = sc + G * scs;
    if (tid < 32) etab[tid] = kExp2Tab[tid];

    // 1. scores, K in chunks of kcap <= T rows
    const float* kbase = kc + loff + kvo;
    float mx[G];
#pragma unroll
    for (int j = 0; j < G; j++) mx[j] = -INFINITY;
    for (uint32_t r0 = 0; r0 < count; r0 += kcap) {
        const uint32_t nr = count - r0 < kcap ? count - r0 : kcap, slots = nr * F;
        __syncthreads();  // q is in place / the previous chunk is consumed
        for (uint32_t base = wave * 64; base < slots; base += T) {
            const uint32_t s = base + lane;
            if (s < slots) {
                const uint32_t r = s / F, u = (s % F) ^ (r % F);
                __builtin_amdgcn_global_load_lds(kbase + (size_t)win_slot(w, n_shared, r0 + r) * kv_dim + 4 * u,
                                                 work + 4 * base, 16, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this lane's LDS loads have landed
        __syncthreads();
        if (tid < nr) {
            const float* kr = work + tid * HS;
            const uint32_t sw = tid % F;
            float acc[G][4];
#pragma unroll
            for (int j = 0; j < G; j++) acc[j][0] = acc[j][1] = acc[j][2] = acc[j][3] = 0.0f;
#pragma unroll
            for (int c = 0; c < (int)F; c += 16) {  // 16 float4 of the row at a time
                constexpr int U = F < 16 ? F : 16;
                float4 kk[U];
#pragma unroll
                for (int u = 0; u < U; u++) kk[u] = *(const float4*)(kr + 4 * ((c + u) ^ sw));
#pragma unroll
                for (int j = 0; j < G; j++) {
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        // the same q for every lane: scalar loads into SGPRs
                        const float4 qq = *(const float4*)(qg + j * HS + 4 * (c + u));
                        acc[j][0] = __builtin_fmaf(qq.x, kk[u].x, acc[j][0]);
                        acc[j][1] = __builtin_fmaf(qq.y, kk[u].y, acc[j][1]);
                        acc[j][2] = __builtin_fmaf(qq.z, kk[u].z, acc[j][2]);
                        acc[j][3] = __builtin_fmaf(qq.w, kk[u].w, acc[j][3]);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < G; j++) {
                // dot.rs:360: (acc0 + acc1) + (acc2 + acc3), then * scale (cpu.rs:609)
                const float sv = ((acc[j][0] + acc[j][1]) + (acc[j][2] + acc[j][3])) * scale;
                sc[j * scs + r0 + tid] = sv;
                mx[j] = fmaxf(mx[j], sv);
            }
        }
    }

    // 2. per-head max (order-free), then exp with it
#pragma unroll
    for (int j = 0; j < G; j++) {
        float m = mx[j];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if (lane == 0) red[wave][j] = m;
    }
    __syncthreads();
    for (uint32_t t = tid; t < G * count; t += T) {
        const uint32_t j = t / count, i = t - j * count;
        float m = red[0][j];
#pragma unroll
        for (uint32_t wv = 1; wv < T / 64; wv++) m = fmaxf(m, red[wv][j]);
        float* p = sc + j * scs + i;
        *p = glibc_expf(*p - m, etab);
    }
    __syncthreads();

    // 3. V slice rows by LDS DMA (unit f = row f / FV, float4 f % FV, at
    // work[4 f]); the first chunk from waves 1.. while wave 0 runs the sums
    const float* vbase = vc + loff + kvo + d0;
    auto v_dma = [&](uint32_t r0, uint32_t nrows, uint32_t wave0) {
        const uint32_t units = nrows * FV;
        for (uint32_t base = (wave - wave0) * 64; base < units; base += T - 64 * wave0) {
            const uint32_t f = base + lane;
            if (f < units) {
                const uint32_t r = f / FV, col = f - r * FV;
                __builtin_amdgcn_global_load_lds(vbase + (size_t)win_slot(w, n_shared, r0 + r) * kv_dim + 4 * col,
                                                 work + 4 * base, 16, 0, 0);
            }
        }
    };
    if (wave > 0) v_dma(0, count < vcap ? count : vcap, 1);
    // softmax sums, left to right: lane j of wave 0 for head j
    if (tid < G) s_sum[tid] = chain_sum(sc + tid * scs, count);
    __syncthreads();
    for (uint32_t t = tid; t < G * count; t += T) {
        const uint32_t j = t / count, i = t - j * count;
        float* p = sc + j * scs + i;
        const float pv = div_rn(*p, s_sum[j]);
        *p = pv;
        // the probabilities stay in `att`, as the reference leaves them
        if (sidx == 0) att[(size_t)row * n_heads * seq_len + (size_t)(h0 + j) * seq_len + i] = pv;
    }

    // 4. out[h][d0 + e] = sum_i p_i * v_i[e], lane (j, e), i in order
    constexpr uint32_t lanes = G * DW;
    const uint32_t j = tid / DW, e = tid % DW;
    const float* pj = sc + (j < G ? j : 0) * scs;
    float o = 0.0f;
    for (uint32_t r0 = 0; r0 < count; r0 += vcap) {
        const uint32_t nrows = count - r0 < vcap ? count - r0 : vcap;
        if (r0 > 0) {  // a window longer than the V capacity: the next chunk
            __syncthreads();  // every lane is done with the previous one
            v_dma(r0, nrows, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid < lanes) {
            const float* pp = pj + r0;
            const float* vv = work + e;
            uint32_t i = 0;
            for (; i + 32 <= nrows; i += 32) {
                float4 p4[8];
                float v[32];
#pragma unroll
                for (int u = 0; u < 8; u++) p4[u] = *(const float4*)(pp + i + 4 * u);
#pragma unroll
                for (int u = 0; u < 32; u++) v[u] = vv[(i + u) * DW];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    o += p4[u].x * v[4 * u];
                    o += p4[u].y * v[4 * u + 1];
                    o += p4[u].z * v[4 * u + 2];
                    o += p4[u].w * v[4 * u + 3];
                }
            }
            for (; i < nrows; i++) o += pp[i] * vv[i * DW];
        }
    }
    if (tid < lanes) {
        const size_t oi = (size_t)row * width + (size_t)(h0 + j) * HS + d0 + e;
        out[oi] = o;
        // DW % 32 == 0: each 32-lane group is one Q8 block of the head output
        if (qo) quant_lane(o, true, qo + oi, so + oi / 32, ho + oi / 32);
    }
}

// ---------------------------------------------------------------------------
// Decode attention, split in two launches so that the KV reads spread over
// many CUs (one CU pulls only ~40 GB/s, so a head's whole K and V through one
// workgroup is the critical path otherwise). Same arithmetic as k_attention.
//
// k_attn_scores, workgroup = (KV head, 64 cache rows): RoPE of the head's
// query heads and of the new key (cpu.rs:274-302, the host-built cos/sin
// table; with qnw / knw given, after their per-head RMSNorm, so that the
// q/k norms of a decode step need no launch of their own), the kv_write of the new key and value (cpu.rs:238-246, by the
// chunk-0 workgroup), then one lane per cache row runs the four-chain dot for
// every query head; the scores go to a scratch row per head, and each
// chunk's maximum per head to a second scratch array.
// The new position's key is taken from LDS, not from the cache being written.
// The key rows are read with P consecutive lanes on each row's P 16-byte
// pieces of one phase (P = 16: 256 contiguous bytes per row, four rows per
// load), then passed through LDS (XOR-swizzled, conflict-free both ways) to
// the lane that owns the row: one lane per row reading its own 16-byte
// pieces spreads every load over 64 cache lines and streams at about two
// thirds of the rate of the same bytes read this way.
template <int G, int HS, bool ROPE, bool NORM = false>
__global__ __launch_bounds__(64) void k_attn_scores(const float* __restrict__ q, const float* __restrict__ kin,
                                                    const float* __restrict__ vin, float* __restrict__ kc,
                                                    float* __restrict__ vc, size_t loff,
                                                    const DevWindow* __restrict__ win, const uint32_t* __restrict__ pos,
                                                    const float2* __restrict__ tab, int interleaved, uint32_t kv_dim,
                                                    float scale, float* __restrict__ sc, uint32_t ss,
                                                    float* __restrict__ mxp, uint32_t ms, uint32_t width,
                                                    const float* __restrict__ qnw, const float* __restrict__ knw,
                                                    float eps) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    constexpr uint32_t F = HS / 4, HALF = HS / 2;
    constexpr uint32_t P = F < 16 ? F : 16, NP = F / P, SPL = 64 / P;  // pieces per phase, phases, rows per load
    static_assert(F % P == 0 && (P & (P - 1)) == 0, "head size");
    __shared__ __align__(16) float qs[G * HS];
    __shared__ __align__(16) float kn[HS];
    __shared__ __align__(16) v4f kt[64 * (P + 1)];  // one phase of the 64 key rows, rows padded by one piece
    __shared__ float s_nsc[G + 1];                   // the heads' RMSNorm scales
    const uint32_t lane = threadIdx.x, hk = blockIdx.x, chunk = blockIdx.y, row = blockIdx.z;
    const uint32_t n_heads = width / HS;
    const DevWindow w = win[row];
    sc += (size_t)row * n_heads * ss;
    mxp += (size_t)row * n_heads * ms;
    const uint32_t n_shared = w.shared_end - w.shared_start;
    const uint32_t count = n_shared + w.slot - w.att_start + 1;
    const uint32_t r0 = chunk * 64;
    if (r0 >= count && (chunk != 0 || !ROPE)) return;
    // the 64 key rows, issued first so that their latency overlaps the q and
    // RoPE loads (the new position's key is replaced below by the one rotated
    // here, so reading its cache slot before the write is harmless); load u
    // of phase h brings piece h * P + lane % P of row SPL * u + lane / P, rows
    // past the window read the window's last row
    const uint32_t i = r0 + lane;
    const bool live = i < count;
    const uint32_t ic = live ? i : count - 1;
    const uint32_t pc = lane % P, pr = lane / P;
    const char* kbase = (const char*)(kc + loff + (size_t)hk * HS);
    // the RoPE operands, loaded ahead of the key rows so that their latency
    // overlaps the keys' (global loads complete in issue order): the raw
    // query heads and new key (element t = lane + 64 u of the G + 1 heads),
    // their norm weights, and the (cos, sin) of the pairs this lane rotates
    constexpr uint32_t NX = ROPE ? ((G + 1) * HS + 63) / 64 : 1, NR = ROPE ? ((G + 1) * HALF + 63) / 64 : 1;
    const float* qh = q + (size_t)row * width + (size_t)hk * G * HS;
    const bool nrm = ROPE && NORM && (qnw != nullptr || knw != nullptr);  // NORM: the instantiation with the norms
    float xr[NX], wr[NX];
    float2 cs[NR];
    if (ROPE) {
        const float2* tr = tab + (size_t)pos[0] * HALF;
#pragma unroll
        for (uint32_t u = 0; u < NX; u++) {
            const uint32_t t = lane + 64 * u, hh = t / HS, e = t - hh * HS;
            const bool in = t < (G + 1) * HS;
            const float* nw = hh < G ? qnw : knw;
            xr[u] = in ? (hh < G ? qh[hh * HS + e] : kin[(size_t)hk * HS + e]) : 0.0f;
            wr[u] = NORM && in && nw != nullptr ? nw[e] : 1.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < NR; u++) {
            const uint32_t t = lane + 64 * u, hh = t / HALF;
            cs[u] = t < (G + 1) * HALF ? tr[t - hh * HALF] : make_float2(0.0f, 0.0f);
        }
    }
    v4f kr[F];
#pragma unroll
    for (uint32_t h = 0; h < NP; h++) {
#pragma unroll
        for (uint32_t u = 0; u < P; u++) {
            const uint32_t ri = min(r0 + SPL * u + pr, count - 1);
            kr[h * P + u] = *(const v4f*)(kbase + ((size_t)win_slot(w, n_shared, ri) * kv_dim + 4 * (P * h + pc)) * 4);
        }
    }
    if (!ROPE) {  // q is already rotated, and every key is in the cache
        for (uint32_t t = lane; t < G * F; t += 64) ((float4*)qs)[t] = ((const float4*)qh)[t];
    }
    if (ROPE) {
        // the raw heads to LDS, with the squares into the key tile (free
        // until the first phase) for the per-head RMSNorm of the query heads
        // (qnw) and of the new key (knw) before the rotation (cpu.rs:647-661,
        // k_qk_norm's arithmetic: one lane per head runs the serial sum);
        // LDS-only barriers, so the key rows stay in flight
        float* sq = (float*)kt;
#pragma unroll
        for (uint32_t u = 0; u < NX; u++) {
            const uint32_t t = lane + 64 * u, hh = t / HS, e = t - hh * HS;
            if (t < (G + 1) * HS) {
                (hh < G ? qs + hh * HS : kn)[e] = xr[u];
                if (nrm) sq[t] = xr[u] * xr[u];
            }
        }
        lds_barrier();
        if (nrm) {
            if (lane <= (uint32_t)G) {
                float sc1 = 1.0f;
                if (lane < (uint32_t)G ? qnw != nullptr : knw != nullptr) {
                    float ssq = chain_sum(sq + lane * HS, HS);
                    ssq = div_rn(ssq, (float)HS);
                    ssq += eps;
                    sc1 = div_rn(1.0f, sqrt_rn(ssq));
                }
                s_nsc[lane] = sc1;
            }
            lds_barrier();
#pragma unroll
            for (uint32_t u = 0; u < NX; u++) {
                const uint32_t t = lane + 64 * u, hh = t / HS, e = t - hh * HS;
                if (t < (G + 1) * HS && (hh < G ? qnw != nullptr : knw != nullptr))
                    (hh < G ? qs + hh * HS : kn)[e] = wr[u] * (s_nsc[hh] * xr[u]);
            }
            lds_barrier();
        }
        // the rotation in place: one lane reads and writes both values of a pair
#pragma unroll
        for (uint32_t u = 0; u < NR; u++) {
            const uint32_t t = lane + 64 * u, hh = t / HALF, e = t - hh * HALF;
            if (t < (G + 1) * HALF) {
                float* dst = hh < G ? qs + hh * HS : kn;
                const uint32_t i0 = interleaved ? 2 * e : e, i1 = interleaved ? 2 * e + 1 : e + HALF;
                const float a = dst[i0], b = dst[i1];
                dst[i0] = a * cs[u].x - b * cs[u].y;
                dst[i1] = a * cs[u].y + b * cs[u].x;
            }
        }
    }
    __syncthreads();
    if (ROPE && chunk == 0) {
        const size_t at = loff + (size_t)w.slot * kv_dim + (size_t)hk * HS;
        for (uint32_t e = lane; e < HS; e += 64) {
            kc[at + e] = kn[e];
            vc[at + e] = vin[(size_t)hk * HS + e];
        }
        if (r0 >= count) return;
    }
    // the four chains of every query head, dims in order (dot.rs:350-366),
    // one phase of P pieces at a time through LDS: piece t of row r sits at
    // r * (P + 1) + t (the padding keeps both the row-wise stores and the
    // lane-per-row reads free of bank conflicts)
    float a[G][4];
#pragma unroll
    for (int j = 0; j < G; j++) a[j][0] = a[j][1] = a[j][2] = a[j][3] = 0.0f;
    const bool fresh = ROPE && ic == count - 1;  // the new position: its key is the one just rotated
#pragma unroll
    for (uint32_t h = 0; h < NP; h++) {
        if (h) __syncthreads();  // the previous phase is read
#pragma unroll
        for (uint32_t u = 0; u < P; u++) {
            const uint32_t r = SPL * u + pr;
            kt[r * (P + 1) + pc] = kr[h * P + u];
        }
        __syncthreads();
        v4f kk[P];
#pragma unroll
        for (uint32_t t = 0; t < P; t++) kk[t] = fresh ? ((const v4f*)kn)[h * P + t] : kt[lane * (P + 1) + t];
        // q (the same for every lane) in groups of Q pieces, each group read
        // while the previous one's FMAs run; the empty asm statements pin that
        // order, so the compiler does not hold every head's q in registers
        constexpr uint32_t Q = P < 4 ? P : 4, NG = G * (P / Q);
        const v4f* qv = (const v4f*)qs + h * P;
        v4f qg[2][Q];
#pragma unroll
        for (uint32_t t = 0; t < Q; t++) qg[0][t] = qv[t];
#pragma unroll
        for (uint32_t g = 0; g < NG; g++) {
            const uint32_t j = g / (P / Q), t0 = (g % (P / Q)) * Q;
            if (g + 1 < NG) {
                const uint32_t jn = (g + 1) / (P / Q), tn = ((g + 1) % (P / Q)) * Q;
#pragma unroll
                for (uint32_t t = 0; t < Q; t++) qg[(g + 1) & 1][t] = qv[jn * F + tn + t];
            }
#pragma unroll
            for (uint32_t t = 0; t < Q; t++) {
                const v4f qq = qg[g & 1][t];
                a[j][0] = __builtin_fmaf(qq.x, kk[t0 + t].x, a[j][0]);
                a[j][1] = __builtin_fmaf(qq.y, kk[t0 + t].y, a[j][1]);
                a[j][2] = __builtin_fmaf(qq.z, kk[t0 + t].z, a[j][2]);
                a[j][3] = __builtin_fmaf(qq.w, kk[t0 + t].w, a[j][3]);
            }
            __asm__ __volatile__("" : "+v"(a[j][0]), "+v"(a[j][1]), "+v"(a[j][2]), "+v"(a[j][3])::"memory");
        }
    }
#pragma unroll
    for (int j = 0; j < G; j++) {
        // dot.rs:360: (acc0 + acc1) + (acc2 + acc3), then * scale (cpu.rs:609)
        const float sv = ((a[j][0] + a[j][1]) + (a[j][2] + a[j][3])) * scale;
        if (live) sc[(size_t)(hk * G + j) * ss + i] = sv;
        // the chunk's maximum (order-free), so the softmax launch need not scan the scores for it
        const float m = wave_max(live ? sv : -INFINITY);
        if (lane == 0) mxp[(size_t)(hk * G + j) * ms + chunk] = m;
    }
}

// k_attn_softmax_v, workgroup = (KV head, DW of its HS output dims), 16
// waves. Every wave reduces the per-chunk maxima of the G heads (written by
// k_attn_scores) while the scores arrive by LDS DMA; all waves run the exp;
// then waves 8-15 issue the loads of the V slice into registers (they land
// while the sum runs); wave j runs head j's serial softmax sum while
// waves 8-15 store the V slice transposed ([dim][position]); all waves
// divide; all waves form every product p_i * v_i[e] (rounded) into a table
// with a row per (query head, dim); then one lane per row runs the weighted V
// sum in position order, a chain of adds whose operands arrive 32 at a time
// (a chain step that also loaded its two operands and multiplied them would
// take about twice as long). The probabilities are left in `att` (slice 0),
// as the reference leaves them.
// LDS: probabilities [G][scs] | V slice [DW][vst] | products [G * DW][vst],
// vst = round64(scs) + 4 (the 16 rows of a transposed read start 16 bytes
// apart, on distinct banks).
static constexpr uint32_t kAttnVRegs = 8;  // V float4 per thread held in registers
__host__ __device__ inline size_t attn_split_vst(size_t pw) { return ((pw + 63) & ~(size_t)63) + 4; }
// pw: the positions of one pass of the V slice and product table (the whole
// window in one pass where that fits)
__host__ __device__ inline size_t attn_split_lds(size_t scs, size_t G, size_t DW, size_t pw) {
    return (G * scs + (DW + G * DW) * attn_split_vst(pw)) * sizeof(float);
}
__host__ __device__ inline size_t attn_split_ms(size_t seq_len) { return ((seq_len + 63) / 64 + 3) & ~(size_t)3; }
template <int G, int HS, int DW, bool LONG = false>
__global__ __launch_bounds__(1024) void k_attn_softmax_v(const float* __restrict__ sc_in, uint32_t ss,
                                                         const float* __restrict__ mxp, uint32_t ms,
                                                         const float* __restrict__ vc, size_t loff,
                                                         const DevWindow* __restrict__ win, uint32_t kv_dim,
                                                         uint32_t seq_len, uint32_t scs, float* __restrict__ att,
                                                         float* __restrict__ out, uint32_t pw) {
    constexpr uint32_t S = HS / DW, FV = DW / 4, T = 1024, TV = 512;
    extern __shared__ __align__(16) float sm[];
    __shared__ float s_sum[G];
    __shared__ uint64_t etab[32];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hk = blockIdx.x / S, sidx = blockIdx.x % S, d0 = sidx * DW, row = blockIdx.y;
    const uint32_t n_heads = gridDim.x / S * G;
    const DevWindow w = win[row];
    sc_in += (size_t)row * n_heads * ss;
    mxp += (size_t)row * n_heads * ms;
    att += (size_t)row * n_heads * seq_len;
    out += (size_t)row * n_heads * HS;
    const uint32_t n_shared = w.shared_end - w.shared_start;
    const uint32_t count = n_shared + w.slot - w.att_start + 1;  // <= scs
    const uint32_t vst = (uint32_t)attn_split_vst(pw), nch = (count + 63) / 64;
    float* ps = sm;
    float* vt = sm + G * scs;
    // 1. the chunk maxima of the G heads (every wave, a lane per chunk; LONG:
    // windows past 4096 positions, 64 chunks apart), the exp table, ...
    float pm[G];
#pragma unroll
    for (int j = 0; j < G; j++) {
        if constexpr (LONG) {
            float m = -INFINITY;
            for (uint32_t c = lane; c < nch; c += 64) m = fmaxf(m, mxp[(size_t)(hk * G + j) * ms + c]);
            pm[j] = m;
        } else {
            pm[j] = lane < nch ? mxp[(size_t)(hk * G + j) * ms + lane] : -INFINITY;
        }
    }
    const uint64_t et = kExp2Tab[tid & 31];
    __asm__ __volatile__("" ::: "memory");
    // ... and the G score rows by LDS DMA (16-byte units; rows padded to a multiple of 4 floats in both places)
    const uint32_t c4 = (count + 3) / 4, srow = scs / 4;
    for (uint32_t base = wave * 64; base < G * srow; base += T) {
        const uint32_t f = base + lane, j = f / srow, u = f - j * srow;
        if (f < G * srow && u < c4)
            __builtin_amdgcn_global_load_lds(sc_in + (size_t)(hk * G + j) * ss + 4 * u, ps + 4 * base, 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x70);  // vmcnt(0) lgkmcnt(0): maxima, scores, exp table
    if (tid < 32) etab[tid] = et;
    float mx[G];
#pragma unroll
    for (int j = 0; j < G; j++) mx[j] = wave_max(pm[j]);
    lds_barrier();  // the scores and the exp table are in LDS
    // 2. exp with the head's max; the G heads of a position together, so a
    // thread's exps are independent chains that overlap
    for (uint32_t i = tid; i < count; i += T) {
        float e[G];
#pragma unroll
        for (int j = 0; j < G; j++) e[j] = ps[j * scs + i];
#pragma unroll
        for (int j = 0; j < G; j++) ps[j * scs + i] = glibc_expf(e[j] - mx[j], etab);
    }
    lds_barrier();
    // waves 8-15: the V slice into registers (unit f = position f / FV,
    // float4 f % FV); it lands while the softmax sum runs (issued before the
    // exp, it held up the exp phase's barrier)
    const float* vbase = vc + loff + (size_t)hk * HS + d0;
    const uint32_t units0 = min(count, pw) * FV, tv = tid - TV;  // the first pass's V units
    float4 vr[kAttnVRegs];
    if (wave >= 8) {
#pragma unroll
        for (int u = 0; u < (int)kAttnVRegs; u++) {
            const uint32_t f = tv + TV * u;
            if (f < units0) {
                const uint32_t r = f / FV, col = f - r * FV;
                vr[u] = *(const float4*)(vbase + (size_t)win_slot(w, n_shared, r) * kv_dim + 4 * col);
            }
        }
    }
    // 3. softmax sum, left to right (elementwise.rs:81-91), one wave per head
    if (wave < G) {  // register-fed across the wave up to 4096 values, else (LONG) one LDS-fed lane
        float sj;
        if constexpr (LONG)
            sj = lane == 0 ? chain_sum(ps + wave * scs, count) : 0.0f;
        else
            sj = wave_chain_sum(ps + wave * scs, count);
        if (lane == 0) s_sum[wave] = sj;
    }
    // 4-5 in passes of pw positions (one pass where the LDS holds the whole
    // window): waves 8-15 store the pass's V slice transposed (the first pass
    // while the softmax sums run), all waves form the pass's probabilities
    // and products, and the chain lanes continue their sums over them
    constexpr uint32_t NL = G * DW;
    float* prod = vt + DW * vst;
    float acc = 0.0f;  // lane tid < NL: the running V sum of (head tid / DW, dim tid % DW)
    float sj[G];
    for (uint32_t p0 = 0; p0 < count; p0 += pw) {
        const uint32_t pn = min(pw, count - p0), units = pn * FV;
        if (wave >= 8) {
            auto put = [&](uint32_t f, float4 v) {
                const uint32_t r = f / FV, c = 4 * (f - r * FV);
                vt[c * vst + r] = v.x, vt[(c + 1) * vst + r] = v.y, vt[(c + 2) * vst + r] = v.z, vt[(c + 3) * vst + r] = v.w;
            };
            uint32_t f0 = tv;
            if (p0 == 0) {
#pragma unroll
                for (int u = 0; u < (int)kAttnVRegs; u++)
                    if (tv + TV * u < units) put(tv + TV * u, vr[u]);
                f0 = tv + TV * kAttnVRegs;
            }
            for (uint32_t f = f0; f < units; f += TV) {  // past the register capacity, and later passes
                const uint32_t r = f / FV, col = f - r * FV;
                put(f, *(const float4*)(vbase + (size_t)win_slot(w, n_shared, p0 + r) * kv_dim + 4 * col));
            }
        }
        __syncthreads();
        // 4. probabilities, the G heads of a position together (elementwise.rs:88-91),
        // and at once the products p_i * v_i[e] of out[h][d0 + e] = sum_i p_i *
        // v_i[e] into row j * DW + e; +0.0 from count to round32(count) (adding
        // +0.0 leaves every reachable running sum unchanged: it starts at +0.0
        // and so is never -0.0)
        const uint32_t n32 = (pn + 31) & ~31u;
#pragma unroll
        for (int j = 0; j < G; j++) sj[j] = s_sum[j];
        for (uint32_t i = tid; i < n32; i += T) {
            const bool live = i < pn;
            const uint32_t ii = live ? i : 0;
            float pv[G], vv[DW];
#pragma unroll
            for (int e = 0; e < (int)DW; e++) vv[e] = vt[e * vst + ii];
#pragma unroll
            for (int j = 0; j < G; j++) pv[j] = div_rn(ps[j * scs + p0 + ii], sj[j]);
#pragma unroll
            for (int j = 0; j < G; j++) {
                if (live) ps[j * scs + p0 + i] = pv[j];
#pragma unroll
                for (int e = 0; e < (int)DW; e++) prod[(j * DW + e) * vst + i] = live ? pv[j] * vv[e] : 0.0f;
            }
        }
        // 5. the chains, i in order
        __syncthreads();
        const bool last = p0 + pw >= count;
        if (tid < NL) {
            acc = chain_sum(prod + tid * vst, n32, acc);
        } else if (last && sidx == 0 && tid >= 64) {
            // the probabilities to `att` while the chains run (global stores
            // issued earlier would hold up every later wait on the memory counter)
            for (uint32_t t = tid - 64; t < G * count; t += T - 64) {
                const uint32_t j = t / count, i = t - j * count;
                att[(size_t)(hk * G + j) * seq_len + i] = ps[j * scs + i];
            }
        }
        if (!last) __syncthreads();  // the chains have read the table before the next pass rewrites it
    }
    if (tid < NL) out[(size_t)(hk * G + tid / DW) * HS + d0 + tid % DW] = acc;
}

static constexpr size_t kAttnSplitLds = 150 * 1024;
// dims per k_attn_softmax_v workgroup: 4 (twice the workgroups of 8, each
// with half the products to form; measured faster)
static constexpr size_t kAttnSplitDW = 4;
// positions per pass of k_attn_softmax_v's V slice and product table: the
// whole window in one pass where the LDS holds it, else the fewest passes
// (of whole 64-position chunks) that fit beside the G score rows; 0: none do
static size_t attn_split_pass(size_t scs, size_t G) {
    for (size_t np = 1; np <= 16; np++) {
        const size_t pw = ((scs + np - 1) / np + 63) & ~(size_t)63;
        if (attn_split_lds(scs, G, kAttnSplitDW, pw) <= kAttnSplitLds) return pw;
    }
    return 0;
}

bool attention_split_ok(size_t max_count, size_t kv_mul, size_t hs) {
    if (kv_mul != 1 && kv_mul != 2 && kv_mul != 3 && kv_mul != 4 && kv_mul != 8) return false;
    if (hs != 32 && hs != 64 && hs != 128) return false;
    const size_t scs = (max_count + 3) & ~(size_t)3;
    return max_count >= 1 && max_count <= 16384 && attn_split_pass(scs, kv_mul) > 0;
}

// k_attn_softmax_v_rows: scores [G][scs] | V [64][HS] in LDS, so the window
// is bounded by what those take (at most 16384 positions)
bool attention_split_rows_ok(size_t max_count, size_t kv_mul, size_t hs) {
    if (kv_mul != 1 && kv_mul != 2 && kv_mul != 3 && kv_mul != 4 && kv_mul != 8) return false;
    if (hs != 32 && hs != 64 && hs != 128) return false;
    const size_t scs = (max_count + 3) & ~(size_t)3;
    return max_count >= 1 && max_count <= 16384 && (kv_mul * scs + 64 * hs) * sizeof(float) <= kAttnSplitLds;
}

// scores [n_heads][round4(seq_len)] | chunk maxima [n_heads][attn_split_ms(seq_len)]
size_t attention_split_scratch(size_t n_heads, size_t seq_len) {
    return n_heads * (((seq_len + 3) & ~(size_t)3) + attn_split_ms(seq_len));
}

hipError_t launch_attention_split(hipStream_t st, const float* q, const float* k, const float* v, float* out,
                                  float* att, float* kc, float* vc, size_t layer, const DevWindow* window,
                                  const uint32_t* pos, const float2* table, int interleaved, size_t max_count,
                                  size_t n_heads, size_t kv_mul, size_t hs, size_t kv_dim, size_t seq_len,
                                  float scale, float* scratch, const float* qnw, const float* knw, float eps) {
    if (!attention_split_ok(max_count, kv_mul, hs) || n_heads % kv_mul != 0 || max_count > seq_len)
        return hipErrorInvalidValue;
    const size_t n_kv = n_heads / kv_mul, nchunks = (max_count + 63) / 64, loff = layer * seq_len * kv_dim;
    const size_t scs = (max_count + 3) & ~(size_t)3;
    float* sc = scratch;
    const uint32_t ss = (uint32_t)((seq_len + 3) & ~(size_t)3);  // scratch row stride
    const uint32_t ms = (uint32_t)attn_split_ms(seq_len);
    float* mxp = scratch + n_heads * ss;
    const size_t pw = attn_split_pass(scs, kv_mul), lds = attn_split_lds(scs, kv_mul, kAttnSplitDW, pw);
    const dim3 g1((unsigned)n_kv, (unsigned)nchunks), g2((unsigned)(n_kv * (hs / kAttnSplitDW)));
#define KR_SPLIT(G, H)                                                                                              \
    do {                                                                                                            \
        if (qnw || knw)                                                                                             \
            hipLaunchKernelGGL((k_attn_scores<G, H, true, true>), g1, dim3(64), 0, st, q, k, v, kc, vc, loff, window, \
                               pos, table, interleaved, (uint32_t)kv_dim, scale, sc, ss, mxp, ms,                   \
                               (uint32_t)(n_heads * hs), qnw, knw, eps);                                            \
        else                                                                                                        \
            hipLaunchKernelGGL((k_attn_scores<G, H, true>), g1, dim3(64), 0, st, q, k, v, kc, vc, loff, window, pos, \
                               table, interleaved, (uint32_t)kv_dim, scale, sc, ss, mxp, ms, (uint32_t)(n_heads * hs), \
                               nullptr, nullptr, 0.0f);                                                             \
        if (max_count > 64 * 64)                                                                                    \
            hipLaunchKernelGGL((k_attn_softmax_v<G, H, kAttnSplitDW, true>), g2, dim3(1024), lds, st, sc, ss, mxp,  \
                               ms, vc, loff, window, (uint32_t)kv_dim, (uint32_t)seq_len, (uint32_t)scs, att, out,  \
                               (uint32_t)pw);                                                                       \
        else                                                                                                        \
            hipLaunchKernelGGL((k_attn_softmax_v<G, H, kAttnSplitDW>), g2, dim3(1024), lds, st, sc, ss, mxp, ms,    \
                               vc, loff, window, (uint32_t)kv_dim, (uint32_t)seq_len, (uint32_t)scs, att, out,      \
                               (uint32_t)pw);                                                                       \
    } while (0)
#define KR_SPLIT_H(G)              \
    if (hs == 32)                  \
        KR_SPLIT(G, 32);           \
    else if (hs == 64)             \
        KR_SPLIT(G, 64);           \
    else                           \
        KR_SPLIT(G, 128);
    switch (kv_mul) {
        case 8: KR_SPLIT_H(8) break;
        case 4: KR_SPLIT_H(4) break;
        case 3: KR_SPLIT_H(3) break;
        case 2: KR_SPLIT_H(2) break;
        default: KR_SPLIT_H(1) break;
    }
#undef KR_SPLIT_H
#undef KR_SPLIT
    return hipGetLastError();
}

// o0 += p[i] * v[i * KS], o1 += p[i] * v[i * KS + 1] for i < n in position
// order (each a rounded product, then a rounded add): p is a 16-byte aligned
// LDS row, v an LDS tile with row stride KS. Batches of kAttnVBatch
// positions in two register sets used in turn (no copies between them): the
// reads of batch b + 1 are issued before the adds of batch b, so the chains
// wait on the previous add rather than on LDS; the last n % kAttnVBatch
// positions run one at a time.
static constexpr uint32_t kAttnVBatch = 8;
template <uint32_t KS>
__device__ __forceinline__ void attn_v_chain(const float* __restrict__ p, const float* __restrict__ v, uint32_t n,
                                             float& o0, float& o1) {
    typedef float v2f __attribute__((ext_vector_type(2)));
    typedef float v4f __attribute__((ext_vector_type(4)));
    constexpr uint32_t B = kAttnVBatch;
    struct Batch {
        v4f pq[B / 4];
        v2f vv[B];
    };
    auto ld = [&](Batch& b, uint32_t i) {
#pragma unroll
        for (uint32_t k = 0; k < B / 4; k++) b.pq[k] = *(const v4f*)(p + i + 4 * k);
#pragma unroll
        for (uint32_t k = 0; k < B; k++) b.vv[k] = *(const v2f*)(v + (i + k) * KS);
    };
    auto apply = [&](const Batch& b) {
#pragma unroll
        for (uint32_t k = 0; k < B; k++) {
            const float pk = b.pq[k / 4][k % 4];
            o0 += pk * b.vv[k].x;
            o1 += pk * b.vv[k].y;
        }
    };
    const uint32_t nb = n / B;  // whole batches
    uint32_t b = 0;
    if (nb > 0) {
        Batch x, y;
        ld(x, 0);
        // x holds batch b; y is loaded with b + 1 before x's adds, and so on
        for (; b + 2 <= nb; b += 2) {
            ld(y, (b + 1) * B);
            apply(x);
            ld(x, (b + 2 < nb ? b + 2 : b + 1) * B);  // past the end: re-read a valid batch, not applied
            apply(y);
        }
        if (b < nb) {
            apply(x);
            b++;
        }
    }
    for (uint32_t i = nb * B; i < n; i++) {
        const float pk = p[i];
        const v2f vk = *(const v2f*)(v + i * KS);
        o0 += pk * vk.x;
        o1 += pk * vk.y;
    }
}

// ---------------------------------------------------------------------------
// Attention for many rows whose windows map positions to the same cache slots
// (prefill: every row of a sequence attends to a prefix of the same slots).
// Same arithmetic as k_attention (cpu.rs:585-632): per (row, head) the 4-chain
// scores, the softmax with its serial sum, the probabilities (left in `att`),
// and per output dim the serial sum over positions of p * v.
//
// Workgroup = (G query heads of one KV head, block of R rows), 8 or 4 waves;
// a (row, head) pair is "rg" = r * G + j, and wave w owns pairs
// w RPW .. w RPW + RPW - 1. Each K tile (64 positions) goes to LDS once and
// serves every pair of the block: lane = position, and the wave's q rows are
// wave-uniform (scalar loads), so one LDS read of 4 K values feeds 4 FMAs per
// pair. The scores stay in LDS; after the last tile each wave runs the max,
// exp, serial sum (one lane per pair) and division of its RPW pairs.
// Then each V tile goes to LDS once and lane (pair, 2 dims)
// runs two independent position-order chains. Row r of the block attends to
// its first count_r positions (its window); the block's windows must agree
// on att_start and the shared range (checked on the host), so window index i
// is the same cache slot for every row.
// LDS: scores [RG][scs] | the current K or V stage (AttnRowsShape::TILE floats).
template <int HS, int NWAVES>
struct AttnRowsShape {
    static constexpr uint32_t NW = NWAVES, NT = 64 * NW;  // waves, threads
    static constexpr uint32_t LPR = HS / 2;          // lanes per pair in the V phase (2 dims each)
    static constexpr uint32_t RPW = 64 / LPR;        // pairs per wave
    static constexpr uint32_t T = 64;                // positions per K tile
    // head_dim 128 stages each tile in two halves (K: half the dims, V: half
    // the positions), which halves the tile's LDS and lets a third
    // workgroup share the CU
    static constexpr uint32_t NH = HS == 128 ? 2 : 1;
    static constexpr uint32_t FK = HS / 4 / NH, KSK = HS / NH + 4;  // K stage: 16-byte columns, row stride
    static constexpr uint32_t TV = T / NH, KSV = HS + 4;           // V stage: positions, row stride
    static constexpr uint32_t TILE = T * KSK > TV * KSV ? T * KSK : TV * KSV;  // floats
};
typedef float attn_v4f __attribute__((ext_vector_type(4)));  // a native vector: stays in registers

// One tile stage of a window into registers: ROWS window positions from i0
// (n of them valid; rows past n re-read row n - 1), C 16-byte columns from
// column c0 of each cache row; thread t holds row t / C + k (NT / C), column
// t % C, for k < PT. Every piece is loaded, so the registers are always
// defined. A whole stage inside one linear run of the window (the shared
// prefix or the own range) takes one slot lookup and a 32-bit byte offset
// per piece.
template <uint32_t C, uint32_t PT, uint32_t NT, uint32_t ROWS>
__device__ __forceinline__ void attn_tile_fetch(attn_v4f (&pre)[PT], const float* base, const DevWindow& w0,
                                                uint32_t n_shared, uint32_t kv_dim, bool off32, uint32_t i0,
                                                uint32_t n, uint32_t c0) {
    constexpr uint32_t RS = NT / C;
    static_assert(NT % C == 0 && PT * RS == ROWS, "tile pieces");
    const uint32_t prow = threadIdx.x / C, pcol = threadIdx.x % C + c0;
    if (off32 && n == ROWS && (i0 + ROWS <= n_shared || i0 >= n_shared)) {
        const char* b = (const char*)base;
        const uint32_t off = (win_slot(w0, n_shared, i0 + prow) * kv_dim + 4 * pcol) * 4;
#pragma unroll
        for (uint32_t k = 0; k < PT; k++) pre[k] = *(const attn_v4f*)(b + off + k * RS * kv_dim * 4);
    } else {
#pragma unroll
        for (uint32_t k = 0; k < PT; k++) {
            const uint32_t rr = prow + k * RS, rc = rr < n ? rr : n - 1;
            pre[k] = *(const attn_v4f*)(base + (size_t)win_slot(w0, n_shared, i0 + rc) * kv_dim + 4 * pcol);
        }
    }
}
// As attn_tile_fetch for a stage of full rows (C = HS / 4 columns from column
// 0), every piece addressed on its own: one code path, so the loads of
// consecutive stages stay independent. n >= 1.
template <uint32_t C, uint32_t PT, uint32_t NT>
__device__ __forceinline__ void attn_tile_fetch_flat(attn_v4f (&pre)[PT], const float* base, const DevWindow& w0,
                                                     uint32_t n_shared, uint32_t kv_dim, uint32_t i0, uint32_t n) {
    constexpr uint32_t RS = NT / C;
    const uint32_t prow = threadIdx.x / C, pcol = threadIdx.x % C;
#pragma unroll
    for (uint32_t k = 0; k < PT; k++) {
        const uint32_t rr = prow + k * RS, rc = rr < n ? rr : n - 1;
        pre[k] = *(const attn_v4f*)(base + (size_t)win_slot(w0, n_shared, i0 + rc) * kv_dim + 4 * pcol);
    }
}
// The fetched stage into the LDS tile (row stride STRIDE floats), rows < n.
template <uint32_t C, uint32_t PT, uint32_t NT, uint32_t ROWS, uint32_t STRIDE>
__device__ __forceinline__ void attn_tile_put(const attn_v4f (&pre)[PT], float* kt, uint32_t n) {
    constexpr uint32_t RS = NT / C;
    const uint32_t prow = threadIdx.x / C, pcol = threadIdx.x % C;
    if (n == ROWS) {
#pragma unroll
        for (uint32_t k = 0; k < PT; k++) *(attn_v4f*)(kt + (prow + k * RS) * STRIDE + 4 * pcol) = pre[k];
    } else {
#pragma unroll
        for (uint32_t k = 0; k < PT; k++)
            if (prow + k * RS < n) *(attn_v4f*)(kt + (prow + k * RS) * STRIDE + 4 * pcol) = pre[k];
    }
}
__host__ __device__ constexpr uint32_t attn_pair_group(uint32_t rg) {
    uint32_t p = rg < 8 ? rg : 8;
    while (p > 1 && rg % p != 0) p--;
    return p == 0 ? 1 : p;
}
// Softmax of k_attn_rows' pairs, each by the wave that computed its scores
// (row rg = wave * RPW + k of sc, s_cnt[rg] values): max, exp, the serial sum
// left to right (elementwise.rs:81-91) and the division; the probabilities go
// back to sc and, unless `att` is null, to `att`, where the reference leaves
// them. Two pairs per wave run side by side: their loops interleaved and
// both sums in one pass (wave_chain_sum2).
template <uint32_t RPW, uint32_t G>
__device__ __forceinline__ void attn_rows_softmax(float* __restrict__ sc, uint32_t scs,
                                                  const uint32_t* __restrict__ s_cnt, float* __restrict__ s_sum,
                                                  const uint64_t* __restrict__ etab, uint32_t wave, uint32_t lane,
                                                  uint32_t RG, float* __restrict__ att, uint32_t r0, uint32_t n_heads,
                                                  uint32_t h0, uint32_t seq_len) {
    if constexpr (RPW == 2) {
        const uint32_t ra = wave * 2, rb = ra + 1;
        const uint32_t na = ra < RG ? s_cnt[ra] : 0, nb = rb < RG ? s_cnt[rb] : 0;
        if (na <= 1024 && nb <= 1024) {  // wave-uniform
            const uint32_t nm = max(na, nb);
            float* ea = sc + ra * scs;
            float* eb = sc + (rb < RG ? rb : ra) * scs;
            float ma = -INFINITY, mb = -INFINITY;
            for (uint32_t i = lane; i < nm; i += 64) {
                if (i < na) ma = fmaxf(ma, ea[i]);
                if (i < nb) mb = fmaxf(mb, eb[i]);
            }
            ma = wave_max(ma);
            mb = wave_max(mb);
#pragma unroll 2
            for (uint32_t i = lane; i < nm; i += 64) {
                if (i < na) ea[i] = glibc_expf(ea[i] - ma, etab);
                if (i < nb) eb[i] = glibc_expf(eb[i] - mb, etab);
            }
            __builtin_amdgcn_wave_barrier();
            const float2 sum = wave_chain_sum2(ea, na, eb, nb);
            __builtin_amdgcn_wave_barrier();
            const uint32_t rA = ra / G, jA = ra - rA * G, rB = rb / G, jB = rb - rB * G;
            // null att: nothing is written back (and no offset is taken from it)
            float* aa = att ? att + (size_t)(r0 + rA) * n_heads * seq_len + (size_t)(h0 + jA) * seq_len : nullptr;
            float* ab = att ? att + (size_t)(r0 + rB) * n_heads * seq_len + (size_t)(h0 + jB) * seq_len : nullptr;
#pragma unroll 2
            for (uint32_t i = lane; i < nm; i += 64) {
                if (i < na) {
                    const float pv = div_rn(ea[i], sum.x);
                    ea[i] = pv;
                    if (aa) aa[i] = pv;
                }
                if (i < nb) {
                    const float pv = div_rn(eb[i], sum.y);
                    eb[i] = pv;
                    if (ab) ab[i] = pv;
                }
            }
            return;
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < RPW; k++) {
        const uint32_t rg = wave * RPW + k, n = rg < RG ? s_cnt[rg] : 0;
        float* e = sc + rg * scs;
        float m = -INFINITY;
        for (uint32_t i = lane; i < n; i += 64) m = fmaxf(m, e[i]);
        m = wave_max(m);
#pragma unroll 4
        for (uint32_t i = lane; i < n; i += 64) e[i] = glibc_expf(e[i] - m, etab);  // independent: 4 in flight
    }
    __builtin_amdgcn_wave_barrier();
    // the wave's pairs one after the other, each a register-fed chain across
    // the wave's lanes
#pragma unroll
    for (uint32_t k = 0; k < RPW; k++) {
        const uint32_t rg = wave * RPW + k;
        if (rg < RG) {  // wave-uniform
            const uint32_t n = s_cnt[rg];
            const float sum = n <= 4096 ? wave_chain_sum(sc + rg * scs, n) : chain_sum(sc + rg * scs, n);
            if (lane == 0) s_sum[rg] = sum;
        }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (uint32_t k = 0; k < RPW; k++) {
        const uint32_t rg = wave * RPW + k;
        if (rg >= RG) continue;
        const uint32_t n = s_cnt[rg], r = rg / G, j = rg - r * G;
        const float sj = s_sum[rg];
        float* e = sc + rg * scs;
        float* arow = att ? att + (size_t)(r0 + r) * n_heads * seq_len + (size_t)(h0 + j) * seq_len : nullptr;
#pragma unroll 4
        for (uint32_t i = lane; i < n; i += 64) {
            const float pv = div_rn(e[i], sj);
            e[i] = pv;
            if (arow) arow[i] = pv;
        }
    }
}

template <int G, int HS, int NWAVES>
__global__ __launch_bounds__(64 * NWAVES) void k_attn_rows(const float* __restrict__ q, float* __restrict__ out,
                                                   float* __restrict__ att, const float* __restrict__ kc,
                                                   const float* __restrict__ vc, size_t loff,
                                                   const DevWindow* __restrict__ windows, uint32_t n_rows,
                                                   uint32_t n_heads, uint32_t kv_mul, uint32_t kv_dim,
                                                   uint32_t seq_len, float scale, uint32_t scs,
                                                   int8_t* __restrict__ qo, float* __restrict__ so,
                                                   uint16_t* __restrict__ ho) {
    using Sh = AttnRowsShape<HS, NWAVES>;
    constexpr uint32_t NW = Sh::NW, NT = Sh::NT, LPR = Sh::LPR, RPW = Sh::RPW, T = Sh::T, F = HS / 4;
    constexpr uint32_t NH = Sh::NH, FK = Sh::FK, KSK = Sh::KSK, TV = Sh::TV, KSV = Sh::KSV;
    constexpr uint32_t R = NW * RPW / G, RG = R * G;
    extern __shared__ __align__(16) float sm[];
    float* sc = sm;             // [RG][scs]
    float* kt = sc + RG * scs;  // K stage [T][KSK] (HS < 128) or V stage [TV][KSV]
    __shared__ uint32_t s_cnt[NW * RPW];
    __shared__ float s_sum[NW * RPW];
    __shared__ uint64_t etab[32];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the last row blocks first: a causal prefill's windows grow with the
    // row, so the longest blocks start first and the short ones fill in behind
    const uint32_t r0 = (gridDim.y - 1 - blockIdx.y) * R;
    const uint32_t nr = min(R, n_rows - r0);
    // query heads h0 .. h0 + G - 1 of KV head h0 / kv_mul (G divides kv_mul)
    const uint32_t width = n_heads * HS, h0 = blockIdx.x * G, kvo = (h0 / kv_mul) * HS;
    const DevWindow w0 = windows[r0];
    const uint32_t n_shared = w0.shared_end - w0.shared_start;

    // the window lengths, the exp table; for HS < 128 the block's q rows go to
    // LDS here, so their load overlaps the window read (pairs past the
    // block's end hold the last valid pair's row)
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    // (every load is issued before any store waits on one)
    float* sq = kt + Sh::TILE;  // [RG][HS] (HS < 128)
    attn_v4f qpiece = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (HS < 128) {
        static_assert(RG * F <= NT, "one q piece per thread");
        const uint32_t nvalid = min(RG, nr * G), f = min(tid, RG * F - 1), rg = f / F, u = f - rg * F;
        const uint32_t rc = min(rg, nvalid - 1), r = rc / G, j = rc - r * G;
        qpiece = *(const attn_v4f*)(q + (size_t)(r0 + r) * width + (h0 + j) * HS + 4 * u);
    }
    const uint32_t wslot = windows[r0 + min(tid / G, nr - 1)].slot;
    const uint64_t et = kExp2Tab[tid & 31];
    if constexpr (HS < 128) {
        if (tid < RG * F) *(attn_v4f*)(sq + (tid / F) * HS + 4 * (tid % F)) = qpiece;
    }
    if (tid < NW * RPW) s_cnt[tid] = tid < RG && tid / G < nr ? n_shared + wslot - w0.att_start + 1 : 0;
    if (tid < 32) etab[tid] = et;
    __syncthreads();
    uint32_t cmax = 0;
    for (uint32_t rg = 0; rg < RG; rg++) cmax = max(cmax, s_cnt[rg]);
    const float* kbase = kc + loff + kvo;
    const float* vbase = vc + loff + kvo;
    // K (HS < 128) and V stages are fetched into registers ahead of their use
    // (PT float4 per thread per stage) and stored to LDS after the previous
    // stage is consumed, so the global latency overlaps the compute; the
    // barrier after the compute waits for LDS only, leaving fetches in flight.
    constexpr uint32_t PT = TV * F / NT;
    static_assert(PT * NT == T * FK && PT * NT == TV * F, "K and V stages hold the same pieces");
    const bool off32 = (uint64_t)seq_len * kv_dim * 4 <= 0xFFFFFFFFull;  // every slot's byte offset fits 32 bits
    auto tile_len = [&](uint32_t i0) { return i0 < cmax ? min(T, cmax - i0) : 0u; };

    // the V lane map of phase 3: lane = (pair, 2 dims)
    typedef float v2f __attribute__((ext_vector_type(2)));
    const uint32_t rgv = wave * RPW + lane / LPR, e0 = 2 * (lane % LPR);
    const uint32_t nv = rgv < RG ? s_cnt[rgv] : 0;
    const float* pp = sc + rgv * scs;
    float o0 = 0.0f, o1 = 0.0f;

    if constexpr (HS == 128) {
        // V stage s: positions s TV .. (one stage ahead in `pre`)
        attn_v4f pre[PT];
        auto vlen = [&](uint32_t i0) { return i0 < cmax ? min(TV, cmax - i0) : 0u; };
        auto vfetch = [&](uint32_t st) {
            attn_tile_fetch<F, PT, NT, TV>(pre, vbase, w0, n_shared, kv_dim, off32, st * TV, vlen(st * TV), 0);
        };
        vfetch(0);  // the first V stage lands while the scores and the softmax run
        // 1. scores. Wave w takes window positions 64 (NW t + w) .. + 63 of round
        // t, lane = position, for every pair of the block: the lane's K row comes
        // from memory straight into registers, KD dims at a time (the next chunk
        // in flight while one is used), and the pairs' q values, the same for
        // every lane, sit in scalar registers QD dims at a time. Each K value
        // feeds one FMA per pair and no K passes through LDS.
        {
            constexpr uint32_t PGS = attn_pair_group(RG);  // pairs per group: the largest divisor of RG up to 8
            static_assert(RG % PGS == 0, "pair groups");
            // q dims per scalar block: a power of two with PGS QD <= 32 registers
            constexpr uint32_t QD = 32 / PGS >= 32 ? 32 : 32 / PGS >= 16 ? 16 : 32 / PGS >= 8 ? 8 : 4;
            constexpr uint32_t KD = HS < 32 ? HS : 32, NKC = HS / KD;  // K chunk dims, chunks per row
            static_assert(KD % QD == 0 && QD % 4 == 0 && HS % KD == 0, "blocks");
            const uint32_t nvalid = min(RG, nr * G);  // pairs past the block's end read the last valid pair
            const uint32_t nround = (cmax + 64 * NW - 1) / (64 * NW);
    #pragma unroll 1
            for (uint32_t t = 0; t < nround; t++) {
                const uint32_t pos = (t * NW + wv) * 64 + lane;
                const uint32_t pc = pos < cmax ? pos : cmax - 1;
                const float* krow = kbase + (size_t)win_slot(w0, n_shared, pc) * kv_dim;
    #pragma unroll 1
                for (uint32_t g0 = 0; g0 < RG; g0 += PGS) {
                    const float* qp[PGS];
    #pragma unroll
                    for (uint32_t k = 0; k < PGS; k++) {
                        const uint32_t rg = min(g0 + k, nvalid - 1), r = rg / G, j = rg - r * G;
                        qp[k] = q + (size_t)(r0 + r) * width + (size_t)(h0 + j) * HS;
                    }
                    float acc[PGS][4];
    #pragma unroll
                    for (uint32_t k = 0; k < PGS; k++) acc[k][0] = acc[k][1] = acc[k][2] = acc[k][3] = 0.0f;
                    // the FMAs of K chunk c (in kk) against the pairs' q, QD dims at a
                    // time; the q offsets pass through an empty asm so that no q
                    // block is loaded before the one in use (all of them at once
                    // would not fit the scalar registers)
                    auto qblocks = [&](const float4(&kk)[KD / 4], uint32_t c) {
    #pragma unroll
                        for (uint32_t d0 = 0; d0 < KD; d0 += QD) {
                            float4 qv[PGS][QD / 4];
    #pragma unroll
                            for (uint32_t k = 0; k < PGS; k++) {
                                uint32_t off = c * KD + d0;
                                asm volatile("" : "+s"(off));
                                const float* qk = qp[k] + off;
    #pragma unroll
                                for (uint32_t u = 0; u < QD / 4; u++) qv[k][u] = *(const float4*)(qk + 4 * u);
                            }
    #pragma unroll
                            for (uint32_t u = 0; u < QD / 4; u++) {
                                const float4 kv = kk[d0 / 4 + u];
    #pragma unroll
                                for (uint32_t k = 0; k < PGS; k++) {
                                    const float4 qq = qv[k][u];
                                    acc[k][0] = __builtin_fmaf(qq.x, kv.x, acc[k][0]);
                                    acc[k][1] = __builtin_fmaf(qq.y, kv.y, acc[k][1]);
                                    acc[k][2] = __builtin_fmaf(qq.z, kv.z, acc[k][2]);
                                    acc[k][3] = __builtin_fmaf(qq.w, kv.w, acc[k][3]);
                                }
                            }
                            __builtin_amdgcn_sched_barrier(0);  // the next q block's loads stay below
                        }
                    };
                    auto kload = [&](float4(&kk)[KD / 4], uint32_t c) {
    #pragma unroll
                        for (uint32_t u = 0; u < KD / 4; u++) kk[u] = *(const float4*)(krow + c * KD + 4 * u);
                    };
                    // chunks in two register sets used in turn: the next chunk is in
                    // flight while one is used
                    float4 ka[KD / 4], kb[KD / 4];
                    kload(ka, 0);
    #pragma unroll 1
                    for (uint32_t c = 0; c < NKC; c += 2) {
                        if (c + 1 < NKC) kload(kb, c + 1);
                        qblocks(ka, c);
                        if (c + 2 < NKC) kload(ka, c + 2);
                        if (c + 1 < NKC) qblocks(kb, c + 1);
                    }
    #pragma unroll
                    for (uint32_t k = 0; k < PGS; k++) {
                        const uint32_t rg = g0 + k;
                        // dot.rs:360: (acc0 + acc1) + (acc2 + acc3), then * scale (cpu.rs:609)
                        if (rg < RG && pos < s_cnt[rg])
                            sc[rg * scs + pos] = ((acc[k][0] + acc[k][1]) + (acc[k][2] + acc[k][3])) * scale;
                    }
                }
            }
        }
        __syncthreads();  // every pair's scores are in LDS

        // 2. softmax of each pair, by the wave that computed its scores
        attn_rows_softmax<RPW, G>(sc, scs, s_cnt, s_sum, etab, wave, lane, RG, att, r0, n_heads, h0, seq_len);

        // 3. out[pair][e] = sum_i p_i * v_i[e] in position order; lane = (pair, 2 dims)
        // the first V stage (every wave is past the last K stage)
        const uint32_t nvs = (cmax + TV - 1) / TV;
        attn_tile_put<F, PT, NT, TV, KSV>(pre, kt, vlen(0));
        __syncthreads();
        for (uint32_t st = 0; st < nvs; st++) {
            const uint32_t i0 = st * TV, nt = vlen(i0);
            if (st + 1 < nvs) vfetch(st + 1);
            const uint32_t lim = nv > i0 ? min(nt, nv - i0) : 0;
            attn_v_chain<KSV>(pp + i0, kt + e0, lim, o0, o1);
            lds_barrier();
            if (st + 1 < nvs) {
                attn_tile_put<F, PT, NT, TV, KSV>(pre, kt, vlen(i0 + TV));
                lds_barrier();
            }
        }
    } else {
        // 1. scores of every (pair, position) of each K tile, staged through LDS.
        // K stages s < nks and then V stages s = nks + i of the same shape
        // (HS < 128: one K stage per 64-position tile, the same pieces as a V
        // stage) flow through two register sets used in turn, each stage
        // fetched two stages before it is stored to LDS: the loads of the next
        // two stages are in flight while one is used, and the first two V
        // stages land while the scores and the softmax run. The loops are
        // unrolled by two so that each set is named statically, and every
        // fetch loads its pieces unconditionally (a fetch past the last stage
        // repeats it), so each store to LDS waits for its own loads only.
        const uint32_t nks = (cmax + T - 1) / T, nst = nks + (cmax + TV - 1) / TV;
        attn_v4f pa[PT], pb[PT];
        auto fetch_into = [&](attn_v4f (&p)[PT], uint32_t s) {
            s = min(s, nst - 1);
            const bool isk = s < nks;
            const uint32_t i0 = (isk ? s : s - nks) * T;
            attn_tile_fetch_flat<F, PT, NT>(p, isk ? kbase : vbase, w0, n_shared, kv_dim, i0, tile_len(i0));
        };
        auto put_stage = [&](const attn_v4f (&p)[PT], uint32_t s) {
            attn_tile_put<F, PT, NT, T, KSK>(p, kt, tile_len((s < nks ? s : s - nks) * T));
        };
        static_assert(NH == 1 && FK == F && KSK == KSV && TV == T, "K and V stages share one shape");
        // this wave's pairs' q rows in LDS (the same address on every lane)
        const float* qrow[RPW];
#pragma unroll
        for (uint32_t k = 0; k < RPW; k++) qrow[k] = sq + min(wv * RPW + k, RG - 1) * HS;
        auto scores = [&](uint32_t st) {
            // lane = position, wave = its RPW pairs: QB float4 of each pair's q
            // at a time, then each LDS read of 4 K values feeds 4 FMAs per pair.
            // K is read a group of GS float4 ahead, into two register sets used
            // in turn, so only LDS reads are waited on inside a block.
            const uint32_t i0 = st * T, nt = tile_len(i0);
            constexpr uint32_t QB = 8 / RPW < 2 ? 2 : 8 / RPW, GS = QB < 4 ? QB : 4, NG = QB / GS;
            static_assert(FK % QB == 0 && QB % GS == 0, "q blocks");
            const uint32_t pos = lane;
            float a[RPW][4];
#pragma unroll
            for (uint32_t k = 0; k < RPW; k++) a[k][0] = a[k][1] = a[k][2] = a[k][3] = 0.0f;
            const float* krow = kt + pos * KSK;
#pragma unroll 1
            for (uint32_t q0 = 0; q0 < FK; q0 += QB) {
                float4 qv[RPW][QB];
#pragma unroll
                for (uint32_t k = 0; k < RPW; k++)
#pragma unroll
                    for (uint32_t u = 0; u < QB; u++) qv[k][u] = *(const float4*)(qrow[k] + 4 * (q0 + u));
                float4 kb[2][GS];
#pragma unroll
                for (uint32_t t = 0; t < GS; t++) kb[0][t] = *(const float4*)(krow + 4 * (q0 + t));
#pragma unroll
                for (uint32_t g = 0; g < NG; g++) {
                    if (g + 1 < NG) {
#pragma unroll
                        for (uint32_t t = 0; t < GS; t++)
                            kb[(g + 1) & 1][t] = *(const float4*)(krow + 4 * (q0 + GS * (g + 1) + t));
                    }
#pragma unroll
                    for (uint32_t t = 0; t < GS; t++) {
                        const float4 kk = kb[g & 1][t];
#pragma unroll
                        for (uint32_t k = 0; k < RPW; k++) {
                            const float4 qq = qv[k][GS * g + t];
                            a[k][0] = __builtin_fmaf(qq.x, kk.x, a[k][0]);
                            a[k][1] = __builtin_fmaf(qq.y, kk.y, a[k][1]);
                            a[k][2] = __builtin_fmaf(qq.z, kk.z, a[k][2]);
                            a[k][3] = __builtin_fmaf(qq.w, kk.w, a[k][3]);
                        }
                    }
                }
            }
#pragma unroll
            for (uint32_t k = 0; k < RPW; k++) {
                const uint32_t rg = wv * RPW + k;
                // dot.rs:360: (acc0 + acc1) + (acc2 + acc3), then * scale (cpu.rs:609)
                if (rg < RG && pos < nt && i0 + pos < s_cnt[rg])
                    sc[rg * scs + i0 + pos] = ((a[k][0] + a[k][1]) + (a[k][2] + a[k][3])) * scale;
            }
        };
        fetch_into(pa, 0);
        fetch_into(pb, 1);
        put_stage(pa, 0);
        __syncthreads();
        fetch_into(pa, 2);
        for (uint32_t st = 0; st < nks; st += 2) {
            scores(st);
            lds_barrier();  // the stage is consumed
            if (st + 1 >= nks) break;
            put_stage(pb, st + 1);
            lds_barrier();
            fetch_into(pb, st + 3);
            scores(st + 1);
            lds_barrier();
            if (st + 2 >= nks) break;
            put_stage(pa, st + 2);
            lds_barrier();
            fetch_into(pa, st + 4);
        }

        // 2. softmax of each pair, by the wave that computed its scores (the
        // probabilities go to `att` at the end, so that no store is pending
        // ahead of the V stages' loads)
        attn_rows_softmax<RPW, G>(sc, scs, s_cnt, s_sum, etab, wave, lane, RG, nullptr, r0, n_heads, h0, seq_len);

        // 3. out[pair][e] = sum_i p_i * v_i[e] in position order; lane = (pair, 2 dims).
        // Stage nks (the first V stage) is in pa when nks is even, else in pb.
        auto vphase = [&](attn_v4f (&p0)[PT], attn_v4f (&p1)[PT]) {
            put_stage(p0, nks);
            __syncthreads();
            fetch_into(p0, nks + 2);
            auto chain = [&](uint32_t sv) {
                const uint32_t i0 = sv * TV, nt = tile_len(i0);
                const uint32_t lim = nv > i0 ? min(nt, nv - i0) : 0;
                attn_v_chain<KSV>(pp + i0, kt + e0, lim, o0, o1);
            };
            const uint32_t nvs = nst - nks;
            for (uint32_t sv = 0; sv < nvs; sv += 2) {
                chain(sv);
                lds_barrier();
                if (sv + 1 >= nvs) break;
                put_stage(p1, nks + sv + 1);
                lds_barrier();
                fetch_into(p1, nks + sv + 3);
                chain(sv + 1);
                lds_barrier();
                if (sv + 2 >= nvs) break;
                put_stage(p0, nks + sv + 2);
                lds_barrier();
                fetch_into(p0, nks + sv + 4);
            }
        };
        if (nks & 1)
            vphase(pb, pa);
        else
            vphase(pa, pb);
        // the probabilities, still in LDS, to `att` (the reference leaves them
        // there; null: the caller has no use for them)
        for (uint32_t k = 0; att && k < RPW; k++) {
            const uint32_t rg = wv * RPW + k;
            if (rg >= RG) break;
            const uint32_t n = s_cnt[rg], r = rg / G, j = rg - r * G;
            const float* e = sc + rg * scs;
            float* arow = att + (size_t)(r0 + r) * n_heads * seq_len + (size_t)(h0 + j) * seq_len;
            for (uint32_t i = lane; i < n; i += 64) arow[i] = e[i];
        }
    }
    const uint32_t r = rgv / G, j = rgv - r * G;
    const bool live = rgv < RG && r < nr;
    const size_t o = (size_t)(r0 + r) * width + (size_t)(h0 + j) * HS + e0;
    if (live) *(v2f*)(out + o) = v2f{o0, o1};
    if (qo) {  // head outputs are whole Q8 blocks (HS % 32 == 0): quantize for o_proj (quant.rs:864-873)
        float m = fmaxf(fmaxf(0.0f, fabsf(o0)), fabsf(o1));
        m = group_max16(m);
        const float d = div_rn(m, 127.0f);
        const float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
        if (live) {
            char2 qq;
            qq.x = q8_round(o0 * inv);
            qq.y = q8_round(o1 * inv);
            *(char2*)(qo + o) = qq;
            if ((lane & 15) == 0) {
                so[o / 32] = d;
                ho[o / 32] = f16_bits(d);
            }
        }
    }
}

// LDS bytes of k_attn_rows for windows of up to max_count positions
static size_t attn_rows_lds(size_t G, size_t hs, size_t max_count, size_t nw) {
    const size_t rpw = 128 / hs, rg = (nw * rpw / G) * G, scs = (max_count + 3) & ~(size_t)3;
    const size_t tile = hs == 128 ? std::max(64 * (hs / 2 + 4), 32 * (hs + 4)) : 64 * (hs + 4);  // AttnRowsShape::TILE
    const size_t qrows = hs < 128 ? rg * hs : 0;  // the q rows (HS < 128)
    return (rg * scs + tile + qrows) * sizeof(float);
}
// Waves per k_attn_rows workgroup: 8 while two workgroups fit a CU's LDS,
// else 4 (half the rows per block) if that lets two fit, else whichever fits
// at all (8 first), else 0 (the kernel does not apply).
static size_t attn_rows_waves(size_t G, size_t hs, size_t max_count) {
    if (hs != 32 && hs != 64 && hs != 128) return 0;
    const bool four = 4 * (128 / hs) / G >= 1;  // at least one row per block
    if (attn_rows_lds(G, hs, max_count, 8) <= 80 * 1024) return 8;
    if (four && attn_rows_lds(G, hs, max_count, 4) <= 80 * 1024) return 4;
    if (attn_rows_lds(G, hs, max_count, 8) <= kAttnLds) return 8;
    if (four && attn_rows_lds(G, hs, max_count, 4) <= kAttnLds) return 4;
    return 0;
}
static size_t attn_rows_group(size_t kv_mul) {  // query heads per workgroup
    for (size_t g : {8, 4, 3, 2})
        if (kv_mul % g == 0) return g;
    return 1;
}

// Softmax and V sums of the many-row split attention: workgroup = (KV head,
// row), G * HS threads, lane (j, e) = one output value. The G score rows and
// their chunk maxima come from k_attn_scores; the max, exp, serial sum (one
// lane per head) and division are as in k_attn_softmax_v; then V streams
// through LDS in tiles of 64 positions and every lane runs its own
// position-order chain. All lanes carry a chain, which suits many rows in
// flight (k_attn_softmax_v instead spreads one row over many CUs). The V
// tiles come through two register sets, each tile fetched two tiles ahead of
// its use, the first two before the softmax starts (so their latency runs
// beside the exps and the serial sums); the loop is unrolled by two so that
// each set is named statically and each wait covers its own loads only.
// Fetches past the window read its last row again (never summed). `att` may
// be null: the probabilities are then not written back.
template <int G, int HS>
__global__ __launch_bounds__(G * HS < 64 ? 64 : G * HS) void k_attn_softmax_v_rows(
    const float* __restrict__ sc_in, uint32_t ss, const float* __restrict__ mxp, uint32_t ms,
    const float* __restrict__ vc, size_t loff, const DevWindow* __restrict__ win, uint32_t kv_dim, uint32_t seq_len,
    uint32_t scs, uint32_t n_heads, float* __restrict__ att, float* __restrict__ out, int8_t* __restrict__ qo,
    float* __restrict__ so, uint16_t* __restrict__ ho) {
    constexpr uint32_t NT = G * HS < 64 ? 64 : G * HS, T = 64, F = HS / 4, PT = (T * F + NT - 1) / NT;
    typedef float v4f __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) float sm[];  // probabilities [G][scs] | V tile [T][HS]
    __shared__ float s_sum[G];
    __shared__ float s_max[G];
    __shared__ uint64_t etab[32];
    const uint32_t tid = threadIdx.x, hk = blockIdx.x, row = blockIdx.y;
    const DevWindow w = win[row];
    const uint32_t n_shared = w.shared_end - w.shared_start;
    const uint32_t count = n_shared + w.slot - w.att_start + 1, nch = (count + 63) / 64;
    sc_in += (size_t)row * n_heads * ss + (size_t)hk * G * ss;
    mxp += (size_t)row * n_heads * ms + (size_t)hk * G * ms;
    // null att: the probabilities are not written back (no offset is taken from it)
    float* const arow = att ? att + (size_t)row * n_heads * seq_len + (size_t)hk * G * seq_len : nullptr;
    const size_t ob = (size_t)row * n_heads * HS + (size_t)hk * G * HS;  // this workgroup's first output
    out += ob;
    float* ps = sm;
    float* vt = sm + G * scs;
    const float* vbase = vc + loff + (size_t)hk * HS;
    // scores, maxima, exp table
    for (uint32_t t = tid; t < G * count; t += NT) {
        const uint32_t j = t / count, i = t - j * count;
        ps[j * scs + i] = sc_in[(size_t)j * ss + i];
    }
    if (tid < G) {
        float m = -INFINITY;
        for (uint32_t c = 0; c < nch; c++) m = fmaxf(m, mxp[(size_t)tid * ms + c]);
        s_max[tid] = m;
    }
    if (tid < 32) etab[tid] = kExp2Tab[tid];
    // V tiles: piece f = (position f / F, float4 f % F) of a 64-position tile
    v4f pa[PT], pb[PT];
    auto fetch = [&](v4f(&buf)[PT], uint32_t i0) {
#pragma unroll
        for (uint32_t k = 0; k < PT; k++) {
            const uint32_t f = min(tid + NT * k, T * F - 1), rr = f / F, u = f - rr * F;
            const uint32_t i = min(i0 + rr, count - 1);
            buf[k] = *(const v4f*)(vbase + (size_t)win_slot(w, n_shared, i) * kv_dim + 4 * u);
        }
    };
    auto put = [&](const v4f(&buf)[PT]) {
#pragma unroll
        for (uint32_t k = 0; k < PT; k++) {
            const uint32_t f = tid + NT * k, rr = f / F, u = f - rr * F;
            if (NT * PT == T * F || f < T * F) *(v4f*)(vt + rr * HS + 4 * u) = buf[k];
        }
    };
    // lane (vj, ve): o += p_i * v_i[ve] of head vj over the tile at i0, in
    // position order (cpu.rs:614-628)
    const uint32_t vj = tid / HS, ve = tid - vj * HS;
    auto vsum = [&](float& acc, const float* pr, uint32_t i0) {
        const uint32_t nt = i0 < count ? min(T, count - i0) : 0u;
#pragma unroll 8
        for (uint32_t ii = 0; ii < nt; ii++) acc += pr[i0 + ii] * vt[ii * HS + ve];
    };
    __syncthreads();
    fetch(pa, 0);
    __builtin_amdgcn_sched_barrier(0);  // all of tile 0's loads before tile 1's: the waits count on that order
    fetch(pb, T);
    // the G heads of a position together: independent exps (and divisions) per thread
    float mj[G];
#pragma unroll
    for (int j = 0; j < G; j++) mj[j] = s_max[j];
    for (uint32_t i = tid; i < count; i += NT) {
        float e[G];
#pragma unroll
        for (int j = 0; j < G; j++) e[j] = ps[j * scs + i];
#pragma unroll
        for (int j = 0; j < G; j++) ps[j * scs + i] = glibc_expf(e[j] - mj[j], etab);
    }
    __syncthreads();
    if (tid < G) s_sum[tid] = chain_sum(ps + tid * scs, count);  // elementwise.rs:81-91
    __syncthreads();
    float sj[G];
#pragma unroll
    for (int j = 0; j < G; j++) sj[j] = s_sum[j];
    for (uint32_t i = tid; i < count; i += NT) {
        float pv[G];
#pragma unroll
        for (int j = 0; j < G; j++) pv[j] = div_rn(ps[j * scs + i], sj[j]);
#pragma unroll
        for (int j = 0; j < G; j++) {
            ps[j * scs + i] = pv[j];
            // the probabilities stay in `att`, as the reference leaves them
            if (arow) arow[(size_t)j * seq_len + i] = pv[j];
        }
    }
    __syncthreads();  // the probabilities are in LDS
    const float* pp = ps + (vj < G ? vj : 0) * scs;
    float o = 0.0f;
    // one exit, at the end of the pair (a window of an odd number of tiles
    // runs one empty sum): every path into the loop head has the same order
    // of loads in flight, tile i0 + 2T's before i0 + 3T's
    for (uint32_t i0 = 0; i0 < count; i0 += 2 * T) {
        put(pa);
        lds_barrier();
        fetch(pa, i0 + 2 * T);
        vsum(o, pp, i0);
        lds_barrier();  // the tile is consumed
        put(pb);
        lds_barrier();
        fetch(pb, i0 + 3 * T);
        vsum(o, pp, i0 + T);
        lds_barrier();
    }
    if (tid < G * HS) out[tid] = o;
    // HS % 32 == 0: each 32-lane group is one Q8 block of the row's output
    if (qo) quant_lane(o, tid < G * HS, qo + ob + tid, so + (ob + tid) / 32, ho + (ob + tid) / 32);
}

// Many rows with windows of their own (batched decode of independent
// sequences): the same two launches, without RoPE and kv_write (q rows are
// already rotated and every key is in the cache), one row per grid z (scores)
// or y (softmax and V). `scratch` holds n_rows * attention_split_scratch floats.
hipError_t launch_attention_split_rows(hipStream_t st, const float* q, float* out, float* att, const float* kc,
                                       const float* vc, size_t layer, const DevWindow* windows, size_t n_rows,
                                       size_t max_count, size_t n_heads, size_t kv_mul, size_t hs, size_t kv_dim,
                                       size_t seq_len, float scale, float* scratch, bool keep_att, int8_t* qo,
                                       float* so, uint16_t* ho) {
    if (n_rows == 0) return hipSuccess;
    if (!attention_split_rows_ok(max_count, kv_mul, hs) || n_heads % kv_mul != 0 || max_count > seq_len ||
        (qo && hs % 32 != 0))
        return hipErrorInvalidValue;
    const size_t n_kv = n_heads / kv_mul, nchunks = (max_count + 63) / 64, loff = layer * seq_len * kv_dim;
    const size_t scs = (max_count + 3) & ~(size_t)3;
    const uint32_t ss = (uint32_t)((seq_len + 3) & ~(size_t)3), ms = (uint32_t)attn_split_ms(seq_len);
    float* sc = scratch;
    float* mxp = scratch + n_rows * n_heads * ss;
    const size_t lds = (kv_mul * scs + 64 * hs) * sizeof(float);
    const dim3 g1((unsigned)n_kv, (unsigned)nchunks, (unsigned)n_rows), g2((unsigned)n_kv, (unsigned)n_rows);
    float* kcw = const_cast<float*>(kc);  // written only by the RoPE form
    float* vcw = const_cast<float*>(vc);
#define KR_SPLIT_ROWS(G, H)                                                                                          \
    do {                                                                                                             \
        hipLaunchKernelGGL((k_attn_scores<G, H, false>), g1, dim3(64), 0, st, q, nullptr, nullptr, kcw, vcw, loff,   \
                           windows, nullptr, nullptr, 0, (uint32_t)kv_dim, scale, sc, ss, mxp, ms,                   \
                           (uint32_t)(n_heads * hs), nullptr, nullptr, 0.0f);                                        \
        hipLaunchKernelGGL((k_attn_softmax_v_rows<G, H>), g2, dim3(G * H < 64 ? 64 : G * H), lds, st, sc, ss, mxp, ms, \
                           vc, loff, windows, (uint32_t)kv_dim, (uint32_t)seq_len, (uint32_t)scs, (uint32_t)n_heads,  \
                           keep_att ? att : nullptr, out, qo, so, ho);                                                \
    } while (0)
#define KR_SPLIT_ROWS_H(G)       \
    if (hs == 32)                \
        KR_SPLIT_ROWS(G, 32);    \
    else if (hs == 64)           \
        KR_SPLIT_ROWS(G, 64);    \
    else                         \
        KR_SPLIT_ROWS(G, 128);
    switch (kv_mul) {
        case 8: KR_SPLIT_ROWS_H(8) break;
        case 4: KR_SPLIT_ROWS_H(4) break;
        case 3: KR_SPLIT_ROWS_H(3) break;
        case 2: KR_SPLIT_ROWS_H(2) break;
        default: KR_SPLIT_ROWS_H(1) break;
    }
#undef KR_SPLIT_ROWS_H
#undef KR_SPLIT_ROWS
    return hipGetLastError();
}

// Whether a block of rows can run k_attn_rows: its windows share att_start
// and the shared range (prefill), checked per block of the kernel's R rows.
bool attention_rows_uniform(const DevWindow* w, size_t n_rows, size_t max_count, size_t kv_mul, size_t hs) {
    const size_t G = attn_rows_group(kv_mul), nw = attn_rows_waves(G, hs, max_count);
    if (n_rows < 2 || nw == 0) return false;
    const size_t R = (nw * (128 / hs)) / G;
    for (size_t r = 0; r < n_rows; r++) {
        const DevWindow& a = w[r - r % R];
        if (a.att_start != w[r].att_start || a.shared_start != w[r].shared_start || a.shared_end != w[r].shared_end)
            return false;
    }
    return true;
}

// LDS budget of the latency-first attention and its shape for one call:
// slice width DW (32 or 64), K chunk and V chunk capacities.
static constexpr size_t kAttnFastLds = 150 * 1024;
struct AttnFastShape {
    bool ok;
    uint32_t dw, scs, kcap, vcap;
    size_t lds;
};
static AttnFastShape attn_fast_shape(size_t max_count, size_t G, size_t hs) {
    AttnFastShape r{false, 0, 0, 0, 0, 0};
    if ((hs != 32 && hs != 64 && hs != 128) || G > 8 || max_count == 0) return r;
    const size_t scs = (max_count + 3) & ~(size_t)3;
    const size_t fixed = G * hs + G * scs;  // floats
    if (fixed * 4 + 32 * hs * 4 > kAttnFastLds) return r;
    const size_t work = kAttnFastLds / 4 - fixed;
    size_t kcap = work / hs;
    if (kcap > kAttnFastThreads) kcap = kAttnFastThreads;
    if (kcap > max_count) kcap = max_count;  // LDS sized to the longest window: more workgroups per CU
    // the widest slice whose V window fits in one chunk; else 32 wide, chunked
    size_t dw = 32, vcap = work / 32;
    if (hs >= 64 && work / 64 >= max_count && G * 64 <= kAttnFastThreads) dw = 64, vcap = work / 64;
    if (G * dw > kAttnFastThreads) return r;
    if (vcap >= max_count)
        vcap = max_count;
    else
        vcap &= ~(size_t)31;  // chunk starts stay 16-byte aligned
    r.ok = true;
    r.dw = (uint32_t)dw;
    r.scs = (uint32_t)scs;
    r.kcap = (uint32_t)kcap;
    r.vcap = (uint32_t)vcap;
    r.lds = (fixed + std::max(kcap * hs, vcap * dw)) * 4;
    return r;
}

hipError_t launch_attention(hipStream_t st, const float* q, float* out, float* att, const float* kc,
                            const float* vc, size_t layer, const DevWindow* windows, size_t n_rows,
                            size_t max_count, size_t n_heads, size_t kv_mul, size_t hs, size_t kv_dim,
                            size_t seq_len, float scale, int8_t* qo, float* so, uint16_t* ho,
                            const DevWindow* host_windows, float* mx_scratch, bool keep_att) {
    if (n_rows == 0) return hipSuccess;
    if (hs == 0 || hs > 256 || hs % 4 != 0 || kv_mul == 0 || n_heads % kv_mul != 0) return hipErrorInvalidValue;
    if (qo && hs % 32 != 0) return hipErrorInvalidValue;
    if (max_count > seq_len) max_count = seq_len;
    if (host_windows && mx_scratch && attention_mx_ok(host_windows, n_rows, max_count, kv_mul, hs)) {
        // blocks of 32 (row, head) pairs on the matrix core (attn_mx.hip)
        return launch_attention_mx(st, q, out, att, kc, vc, layer, windows, n_rows, max_count, n_heads, kv_mul, hs,
                                   kv_dim, seq_len, scale, qo, so, ho, mx_scratch, keep_att);
    }
    if (host_windows && attention_rows_uniform(host_windows, n_rows, max_count, kv_mul, hs)) {
        // many rows whose blocks share a window layout: k_attn_rows
        const size_t G = attn_rows_group(kv_mul), nw = attn_rows_waves(G, hs, max_count);
        const size_t R = (nw * (128 / hs)) / G;  // rows per block: AttnRowsShape
        const size_t lds = attn_rows_lds(G, hs, max_count, nw);
        const uint32_t scs = (uint32_t)((max_count + 3) & ~(size_t)3);
        const dim3 grid((unsigned)(n_heads / G), (unsigned)((n_rows + R - 1) / R));
#define KR_ATTN_ROWS(g, h, w)                                                                                 \
    hipLaunchKernelGGL((k_attn_rows<g, h, w>), grid, dim3(64 * w), lds, st, q, out, keep_att ? att : nullptr, kc,   \
                       vc, layer * seq_len * kv_dim, windows, (uint32_t)n_rows, (uint32_t)n_heads,              \
                       (uint32_t)kv_mul, (uint32_t)kv_dim, (uint32_t)seq_len, scale, scs, qo, so, ho)
#define KR_ATTN_ROWS_W(g, h)         \
    if (nw == 8)                     \
        KR_ATTN_ROWS(g, h, 8);       \
    else                             \
        KR_ATTN_ROWS(g, h, 4);
#define KR_ATTN_ROWS_G(g)          \
    if (hs == 32)                  \
        KR_ATTN_ROWS_W(g, 32)      \
    else if (hs == 64)             \
        KR_ATTN_ROWS_W(g, 64)      \
    else                           \
        KR_ATTN_ROWS_W(g, 128)
        switch (G) {
            case 8: KR_ATTN_ROWS_G(8) break;
            case 4: KR_ATTN_ROWS_G(4) break;
            case 3: KR_ATTN_ROWS_G(3) break;
            case 2: KR_ATTN_ROWS_G(2) break;
            default: KR_ATTN_ROWS_G(1) break;
        }
#undef KR_ATTN_ROWS_G
#undef KR_ATTN_ROWS_W
#undef KR_ATTN_ROWS
        return hipGetLastError();
    }
    {
        // heads per workgroup: the largest of 8, 4, 3, 2, 1 dividing kv_mul
        size_t G = 1;
        for (size_t g : {8, 4, 3, 2})
            if (kv_mul % g == 0) {
                G = g;
                break;
            }
        const AttnFastShape f = attn_fast_shape(max_count, G, hs);
        if (f.ok) {
            const dim3 grid((unsigned)(n_heads / G * (hs / f.dw)), (unsigned)n_rows);
#define KR_ATTN_FAST(g, h, d)                                                                                    \
    hipLaunchKernelGGL((k_attention_fast<g, h, d>), grid, dim3(kAttnFastThreads), f.lds, st, q, out, att, kc, vc, \
                       layer * seq_len * kv_dim, windows, (uint32_t)n_heads, (uint32_t)kv_mul, (uint32_t)kv_dim,  \
                       (uint32_t)seq_len, scale, f.scs, f.kcap, f.vcap, qo, so, ho)
#define KR_ATTN_FAST_G(g)                   \
    if (hs == 32)                           \
        KR_ATTN_FAST(g, 32, 32);            \
    else if (hs == 64 && f.dw == 32)        \
        KR_ATTN_FAST(g, 64, 32);            \
    else if (hs == 64)                      \
        KR_ATTN_FAST(g, 64, 64);            \
    else if (f.dw == 32)                    \
        KR_ATTN_FAST(g, 128, 32);           \
    else                                    \
        KR_ATTN_FAST(g, 128, 64);
            switch (G) {
                case 8: KR_ATTN_FAST_G(8) break;
                case 4: KR_ATTN_FAST_G(4) break;
                case 3: KR_ATTN_FAST_G(3) break;
                case 2: KR_ATTN_FAST_G(2) break;
                default: KR_ATTN_FAST_G(1) break;
            }
#undef KR_ATTN_FAST_G
#undef KR_ATTN_FAST
            return hipGetLastError();
        }
    }
    size_t G = 1;  // heads per workgroup: the largest divisor of kv_mul that fits
    for (size_t g = 1; g <= 8 && g <= kv_mul; g++)
        if (kv_mul % g == 0 && g * hs <= 2 * kAttnThreads) G = g;
    size_t qn = G * hs;
    size_t qbytes = ((qn + 3) & ~(size_t)3) * sizeof(float);
    // V tiles: as many rows as the window needs, at most 8 float4 per lane
    size_t tile_rows = (8 * 4 * kAttnThreads) / hs;
    size_t need_rows = max_count < tile_rows ? max_count : tile_rows;
    if (need_rows < 1) need_rows = 1;
    size_t vbytes = 2 * need_rows * hs * sizeof(float);
    size_t lds_scores = qbytes + vbytes + G * max_count * sizeof(float) <= kAttnLds ? max_count : 0;
    size_t lds = qbytes + vbytes + G * lds_scores * sizeof(float);
    hipLaunchKernelGGL(k_attention, dim3((unsigned)(n_heads / G), (unsigned)n_rows), dim3(kAttnThreads), lds, st, q,
                       out, att, kc, vc, layer * seq_len * kv_dim, windows, (uint32_t)n_heads, (uint32_t)kv_mul,
                       (uint32_t)hs, (uint32_t)kv_dim, (uint32_t)seq_len, scale, (uint32_t)G, (uint32_t)lds_scores,
                       (uint32_t)need_rows, qo, so, ho);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fused steps of the model driver. Each reproduces, in one launch, the exact
// arithmetic of a short run of separate ops.

// add_in_place (cpu.rs:405-410) + rms_norm (cpu.rs:633-644) + the Q8
// quantization of the normed row (quant.rs:856-874), one row per workgroup.
// Thread t holds float4 t, t + 256, ... of the row in registers: the residual
// sum, the norm weight (loaded before the chain, off its critical path) and
// the squares, which go to LDS for the serial sum. Lane 0 alone runs that
// sum, reading LDS in runs of 64 values per wait (one active lane: the same
// loop on all 64 lanes of a wave ran 2.5x slower when other work shared the
// CU). A Q8 block is 8 consecutive threads.
// pstride > 0: `add` is four partial-sum planes of a chain-split projection,
// pstride floats apart, added as ((p0 + p1) + p2) + p3 (dot.rs:45) before the
// residual add. cm: the Q8 blocks go out in chain-major order (cm_block).
template <bool ADD, int VPT>
__global__ __launch_bounds__(256) void k_add_rms_quant(float* __restrict__ x, const float* __restrict__ add,
                                                       const float* __restrict__ w, float* __restrict__ out,
                                                       uint32_t dim, float eps, int8_t* __restrict__ q,
                                                       float* __restrict__ s, uint16_t* __restrict__ h,
                                                       size_t pstride, uint32_t cm) {
    extern __shared__ __align__(16) float sq[];  // [dim]
    __shared__ float s_scale;
    const uint32_t tid = threadIdx.x, n4 = dim / 4;
    const size_t row = blockIdx.x;
    float4* xr = (float4*)(x + row * dim);
    float4 v[VPT], wv[VPT];
#pragma unroll
    for (int u = 0; u < VPT; u++) {
        const uint32_t f = tid + 256 * u;
        if (f < n4) {
            v[u] = xr[f];
            wv[u] = ((const float4*)w)[f];
            if (ADD) {
                float4 a = ((const float4*)(add + row * dim))[f];
                if (pstride) {
                    const float4 a1 = ((const float4*)(add + pstride + row * dim))[f];
                    const float4 a2 = ((const float4*)(add + 2 * pstride + row * dim))[f];
                    const float4 a3 = ((const float4*)(add + 3 * pstride + row * dim))[f];
                    a = make_float4(((a.x + a1.x) + a2.x) + a3.x, ((a.y + a1.y) + a2.y) + a3.y,
                                    ((a.z + a1.z) + a2.z) + a3.z, ((a.w + a1.w) + a2.w) + a3.w);
                }
                v[u] = make_float4(v[u].x + a.x, v[u].y + a.y, v[u].z + a.z, v[u].w + a.w);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < VPT; u++) {
        const uint32_t f = tid + 256 * u;
        if (f < n4) {
            if (ADD) xr[f] = v[u];
            ((float4*)sq)[f] = make_float4(v[u].x * v[u].x, v[u].y * v[u].y, v[u].z * v[u].z, v[u].w * v[u].w);
        }
    }
    __syncthreads();
    // rms_norm_row (cpu.rs:635-641): ss = sum of squares left to right (in its
    // exact parallel form), ss /= dim, ss += eps, scale = 1 / sqrt(ss)
    float ss = rms_sum4(sq, dim);
    if (tid < 64) {
        ss = div_rn(ss, (float)dim);
        ss += eps;
        if (tid == 0) s_scale = div_rn(1.0f, sqrt_rn(ss));
    }
    __syncthreads();
    const float scale = s_scale;
    const uint32_t nb = dim / 32;
#pragma unroll
    for (int u = 0; u < VPT; u++) {
        const uint32_t f = tid + 256 * u;
        // dim % 32 == 0: the 8 threads of a block are all in range or all out
        if (f < n4) {
            // cpu.rs:643: out = w * (scale * x)
            const float4 o = make_float4(wv[u].x * (scale * v[u].x), wv[u].y * (scale * v[u].y),
                                         wv[u].z * (scale * v[u].z), wv[u].w * (scale * v[u].w));
            ((float4*)(out + row * dim))[f] = o;
            // Q8Vec::quantize_into (quant.rs:864-873) on the block of 8 threads
            float m = fmaxf(fmaxf(fmaxf(fmaxf(0.0f, fabsf(o.x)), fabsf(o.y)), fabsf(o.z)), fabsf(o.w));
            m = group_max8(m);
            const float d = div_rn(m, 127.0f);
            const float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
            char4 qq;
            qq.x = q8_round(o.x * inv);
            qq.y = q8_round(o.y * inv);
            qq.z = q8_round(o.z * inv);
            qq.w = q8_round(o.w * inv);
            const uint32_t pb = cm ? cm_block(f / 8, nb) : f / 8;
            ((char4*)(q + row * dim + pb * 32))[f & 7] = qq;
            if ((f & 7) == 0) {
                s[row * nb + pb] = d;
                h[row * nb + pb] = f16_bits(d);
            }
        }
    }
}

hipError_t launch_add_rms_quant(hipStream_t st, float* x, const float* add, const float* w, float* out,
                                size_t rows, size_t dim, float eps, int8_t* q, float* s, uint16_t* h, int add_planes,
                                bool chain_major) {
    if (rows == 0) return hipSuccess;
    if (dim % 32 != 0 || dim > 8192 || (add_planes != 1 && add_planes != 4) || (chain_major && dim % 128 != 0))
        return hipErrorInvalidValue;
    const size_t pstride = add_planes == 4 ? rows * dim : 0;
    const uint32_t cm = chain_major ? 1u : 0u;
    const size_t lds = dim * sizeof(float);
    const size_t vpt = (dim / 4 + 255) / 256;
#define KR_NORM_GO(A, V)                                                                                        \
    hipLaunchKernelGGL((k_add_rms_quant<A, V>), dim3((unsigned)rows), dim3(256), lds, st, x, add, w, out,      \
                       (uint32_t)dim, eps, q, s, h, pstride, cm)
#define KR_NORM_V(A)          \
    if (vpt <= 1)             \
        KR_NORM_GO(A, 1);     \
    else if (vpt <= 2)        \
        KR_NORM_GO(A, 2);     \
    else if (vpt <= 4)        \
        KR_NORM_GO(A, 4);     \
    else                      \
        KR_NORM_GO(A, 8);
    if (add) {
        KR_NORM_V(true)
    } else {
        KR_NORM_V(false)
    }
#undef KR_NORM_V
#undef KR_NORM_GO
    return hipGetLastError();
}

// silu_mul (cpu.rs:494-499) + quantization of the gated rows.
__global__ __launch_bounds__(256) void k_silu_quant(float* __restrict__ g, const float* __restrict__ u, size_t n,
                                                    int8_t* __restrict__ q, float* __restrict__ s,
                                                    uint16_t* __restrict__ h) {
    __shared__ uint64_t etab[32];  // the exp table in LDS: per-lane lookups without a global round trip
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    bool valid = i < n;  // n % 32 == 0
    const float xv = valid ? g[i] : 0.0f, uv = valid ? u[i] : 0.0f;
    if (threadIdx.x < 32) etab[threadIdx.x] = kExp2Tab[threadIdx.x];
    __syncthreads();
    float r = 0.0f;
    if (valid) {
        r = div_rn(xv, 1.0f + glibc_expf(-xv, etab)) * uv;
        g[i] = r;
    }
    quant_lane(r, valid, q + i, s + i / 32, h + i / 32);
}

hipError_t launch_silu_quant(hipStream_t st, float* g, const float* u, size_t rows, size_t width, int8_t* q,
                             float* s, uint16_t* h) {
    size_t n = rows * width;
    if (n == 0) return hipSuccess;
    if (width % 32 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_silu_quant, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, n, q, s, h);
    return hipGetLastError();
}

// rope (cpu.rs:274-302) then kv_write (cpu.rs:238-246): each lane rotates one
// q or k pair and writes rotated k pairs into the cache; v is copied as is.
__global__ __launch_bounds__(256) void k_rope_kv(float* __restrict__ q, float* __restrict__ k,
                                                 const float* __restrict__ v, uint32_t qw, uint32_t kvw,
                                                 uint32_t rows, const uint32_t* __restrict__ pos,
                                                 const uint32_t* __restrict__ slots,
                                                 const float2* __restrict__ tab, uint32_t hs, int interleaved,
                                                 float* __restrict__ kc, float* __restrict__ vc, size_t base) {
    const uint32_t half = hs / 2;
    const uint32_t qpairs = interleaved ? qw / 2 : (qw / hs) * half;
    const uint32_t kpairs = interleaved ? kvw / 2 : (kvw / hs) * half;
    const uint32_t per_row = qpairs + kpairs + kvw;
    uint32_t id = blockIdx.x * 256 + threadIdx.x;
    if (id >= rows * per_row) return;
    uint32_t row = id / per_row, p = id % per_row;
    float* crow_k = kc + base + (size_t)slots[row] * kvw;
    if (p >= qpairs + kpairs) {  // v copy
        uint32_t e = p - qpairs - kpairs;
        vc[base + (size_t)slots[row] * kvw + e] = v[(size_t)row * kvw + e];
        return;
    }
    const float2* tr = tab + (size_t)pos[row] * half;
    bool is_k = p >= qpairs;
    uint32_t pp = is_k ? p - qpairs : p;
    float* vec = is_k ? k + (size_t)row * kvw : q + (size_t)row * qw;
    uint32_t i0, i1;
    float2 cs;
    if (interleaved) {
        i0 = 2 * pp;
        i1 = i0 + 1;
        cs = tr[(i0 % hs) / 2];
    } else {
        uint32_t head = pp / half, i = pp % half;
        i0 = head * hs + i;
        i1 = i0 + half;
        cs = tr[i];
    }
    float a = vec[i0], b = vec[i1];
    float r0 = a * cs.x - b * cs.y;
    float r1 = a * cs.y + b * cs.x;
    vec[i0] = r0;
    vec[i1] = r1;
    if (is_k) {
        crow_k[i0] = r0;
        crow_k[i1] = r1;
    }
}

// Per-head RMSNorm of q and k (cpu.rs:647-661, as k_qk_norm), then their
// RoPE (as k_rope_kv), then k and v into the cache at slots[row]: the three
// steps of a layer with q and k norms in one launch. LP lanes per item (an
// item is one (row, head) of q, of k or of v, which is only copied): 4 for
// a prefill's many items, so that a wave runs 16 of the serial sums side by
// side, 16 for a few rows (a batched-decode step), so that the launch still
// spreads over the CUs:
// the lanes load the head in 16-byte pieces and put the squares in an LDS
// row, the item's first lane runs the serial sum, the normalized values
// replace the squares, each lane rotates its pairs in place (a pair's two
// values are read and written by one lane only), and the lanes store the
// head from LDS in 16-byte pieces.
template <uint32_t LP>
__global__ __launch_bounds__(256) void k_qk_norm_rope_kv(float* __restrict__ q, float* __restrict__ k,
                                                         const float* __restrict__ v, uint32_t qh, uint32_t kh,
                                                         uint32_t rows, uint32_t hs, const float* __restrict__ wq,
                                                         const float* __restrict__ wk, float eps,
                                                         const uint32_t* __restrict__ pos,
                                                         const uint32_t* __restrict__ slots,
                                                         const float2* __restrict__ tab, int interleaved,
                                                         float* __restrict__ kc, float* __restrict__ vc, size_t base) {
    constexpr uint32_t ITEMS = 256 / LP, MAXV4 = 128 / 4 / LP;  // 16-byte pieces per lane: head <= 128
    extern __shared__ __align__(16) float sq[];                   // [ITEMS][hs + 4]
    __shared__ float s_scale[ITEMS];
    const uint32_t slot = threadIdx.x / LP, l = threadIdx.x % LP;
    const uint32_t stride = ((hs + 3) & ~3u) + 4, per_row = qh + 2 * kh, h4 = hs / 4;
    const uint32_t item = blockIdx.x * ITEMS + slot;
    const bool live = item < rows * per_row;
    const uint32_t row = live ? item / per_row : 0, hd = live ? item % per_row : 0;
    const uint32_t kvw = kh * hs;
    if (hd >= qh + kh) {  // v: copied into the cache
        const uint32_t e0 = (hd - qh - kh) * hs;
        float4* cv = (float4*)(vc + base + (size_t)slots[row] * kvw + e0);
        const float4* src = (const float4*)(v + (size_t)row * kvw + e0);
        for (uint32_t i = l; live && i < h4; i += LP) cv[i] = src[i];
        return;  // the item's lanes leave together; only wave-level ordering follows for the others
    }
    const bool is_k = hd >= qh;
    float* vec = is_k ? k + (size_t)row * kvw + (size_t)(hd - qh) * hs : q + (size_t)row * qh * hs + (size_t)hd * hs;
    const float* w = is_k ? wk : wq;
    float* rowl = sq + slot * stride;
    float4 a[MAXV4];
#pragma unroll
    for (uint32_t t = 0; t < MAXV4; t++) {
        const uint32_t i = l + LP * t;
        a[t] = live && i < h4 ? ((const float4*)vec)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < h4) ((float4*)rowl)[i] = make_float4(a[t].x * a[t].x, a[t].y * a[t].y, a[t].z * a[t].z, a[t].w * a[t].w);
    }
    __builtin_amdgcn_wave_barrier();  // an item's lanes are in one wave: LDS order within the wave suffices
    if (l == 0) {  // rms of the head (cpu.rs:635-641 on one head)
        float ss = chain_sum(rowl, hs);
        ss = div_rn(ss, (float)hs);
        ss += eps;
        s_scale[slot] = div_rn(1.0f, sqrt_rn(ss));
    }
    __builtin_amdgcn_wave_barrier();
    const float scale = s_scale[slot];
#pragma unroll
    for (uint32_t t = 0; t < MAXV4; t++) {
        const uint32_t i = l + LP * t;
        if (i < h4) {
            const float4 wv = ((const float4*)w)[i];
            ((float4*)rowl)[i] = make_float4(wv.x * (scale * a[t].x), wv.y * (scale * a[t].y),
                                             wv.z * (scale * a[t].z), wv.w * (scale * a[t].w));
        }
    }
    __builtin_amdgcn_wave_barrier();
    // RoPE of the normalized head (cpu.rs:664-705): pair p is (p, p + half),
    // or (2p, 2p + 1) interleaved; two products and a difference/sum, unfused
    const uint32_t half = hs / 2;
    const float2* tr = tab + (size_t)pos[row] * half;
    for (uint32_t pi = l; pi < half; pi += LP) {
        const uint32_t i0 = interleaved ? 2 * pi : pi, i1 = interleaved ? 2 * pi + 1 : pi + half;
        const float2 cs = tr[pi];
        const float x0 = rowl[i0], x1 = rowl[i1];
        rowl[i0] = x0 * cs.x - x1 * cs.y;
        rowl[i1] = x0 * cs.y + x1 * cs.x;
    }
    __builtin_amdgcn_wave_barrier();
    float4* ck = (float4*)(kc + base + (size_t)slots[row] * kvw + (size_t)(is_k ? hd - qh : 0) * hs);
    for (uint32_t i = l; live && i < h4; i += LP) {
        const float4 r = ((const float4*)rowl)[i];
        ((float4*)vec)[i] = r;
        if (is_k) ck[i] = r;
    }
}

hipError_t launch_qk_norm_rope_kv(hipStream_t st, float* q, float* k, const float* v, size_t qw, size_t kvw,
                                  size_t rows, const float* wq, const float* wk, float eps,
                                  const uint32_t* positions, const uint32_t* slots, const float2* table,
                                  size_t head_size, int interleaved, float* kc, float* vc, size_t layer,
                                  size_t seq_len) {
    if (head_size == 0 || head_size > 128 || head_size % 4 || qw % head_size || kvw % head_size)
        return hipErrorInvalidValue;
    const size_t n = rows * (qw / head_size + 2 * (kvw / head_size));
    if (n == 0) return hipSuccess;
    const size_t stride = head_size + 4;
    // 4 lanes an item where that still leaves 512 or more workgroups
    const bool four = n >= 512 * 64;
    const size_t items = four ? 64 : 16;
    hipLaunchKernelGGL(four ? k_qk_norm_rope_kv<4> : k_qk_norm_rope_kv<16>, dim3((unsigned)((n + items - 1) / items)),
                       dim3(256), items * stride * sizeof(float), st,
                       q, k, v, (uint32_t)(qw / head_size), (uint32_t)(kvw / head_size), (uint32_t)rows,
                       (uint32_t)head_size, wq, wk, eps, positions, slots, table, interleaved, kc, vc,
                       layer * seq_len * kvw);
    return hipGetLastError();
}

hipError_t launch_rope_kv(hipStream_t st, float* q, float* k, const float* v, size_t qw, size_t kvw, size_t rows,
                          const uint32_t* positions, const uint32_t* slots, const float2* table, size_t hs,
                          int interleaved, float* kc, float* vc, size_t layer, size_t seq_len) {
    size_t half = hs / 2;
    size_t per_row = interleaved ? qw / 2 + kvw / 2 + kvw : (qw / hs) * half + (kvw / hs) * half + kvw;
    size_t n = rows * per_row;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_kv, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, q, k, v, (uint32_t)qw,
                       (uint32_t)kvw, (uint32_t)rows, positions, slots, table, (uint32_t)hs, interleaved, kc, vc,
                       layer * seq_len * kvw);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Elementwise ops.
__global__ void k_add(float* __restrict__ d, const float* __restrict__ s, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) d[i] += s[i];
}
hipError_t launch_add(hipStream_t st, float* d, const float* s, size_t n) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, d, s, n);
    return hipGetLastError();
}

// d += ((p0 + p1) + p2) + p3 over the four partial-sum planes of a
// chain-split projection, n floats each (dot.rs:45, then the residual add)
__global__ void k_add_planes(float* __restrict__ d, const float* __restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) d[i] = d[i] + (((p[i] + p[n + i]) + p[2 * n + i]) + p[3 * n + i]);
}
hipError_t launch_add_planes(hipStream_t st, float* d, const float* p, size_t n) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_add_planes, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, d, p, n);
    return hipGetLastError();
}

__global__ void k_mul(float* o, const float* a, const float* b, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        float x = a[i], y = b[i];
        o[i] = x * y;
    }
}
// Overlapping output/input ranges at different offsets: the reference reads
// and writes element by element in order (cpu.rs:424-431), which only a
// sequential loop reproduces.
__global__ void k_mul_seq(float* o, const float* a, const float* b, size_t n) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    for (size_t i = 0; i < n; i++) {
        float x = a[i], y = b[i];
        o[i] = x * y;
    }
}
hipError_t launch_mul(hipStream_t st, float* o, const float* a, const float* b, size_t n, int sequential) {
    if (n == 0) return hipSuccess;
    if (sequential)
        hipLaunchKernelGGL(k_mul_seq, dim3(1), dim3(64), 0, st, o, a, b, n);
    else
        hipLaunchKernelGGL(k_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, o, a, b, n);
    return hipGetLastError();
}

// rows x n products o[r os + i] = a[r as + i] * b[r bs + i] in one launch:
// the per-row mul calls of a batched LFM2 conv layer (lfm2.rs:584-622), whose
// outputs never overlap their inputs
__global__ void k_mul_rows(float* __restrict__ o, size_t os, const float* __restrict__ a, size_t as,
                           const float* __restrict__ b, size_t bs, size_t rows, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * n) return;
    const size_t r = i / n, e = i - r * n;
    const float x = a[r * as + e], y = b[r * bs + e];
    o[r * os + e] = x * y;
}
hipError_t launch_mul_rows(hipStream_t st, float* o, size_t os, const float* a, size_t as, const float* b, size_t bs,
                           size_t rows, size_t n) {
    if (rows * n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_mul_rows, dim3((unsigned)((rows * n + 255) / 256)), dim3(256), 0, st, o, os, a, as, b, bs,
                       rows, n);
    return hipGetLastError();
}

__global__ void k_copy(float* __restrict__ d, const float* __restrict__ s, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) d[i] = s[i];
}
hipError_t launch_copy(hipStream_t st, float* d, const float* s, size_t n) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_copy, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, d, s, n);
    return hipGetLastError();
}

// A bare streaming read, the practical ceiling a read-dominated kernel of the
// same size can reach: CPL 16-byte loads per lane per round, issued
// together, over rounds of 256 CPL pieces per workgroup (a grid-stride loop
// when the grid is smaller than the data), folded into a value that is
// stored only if it matches an impossible pattern.
template <int CPL>
__global__ __launch_bounds__(256) void k_stream_read(const v4i* __restrict__ p, size_t n16, int* __restrict__ sink) {
    v4i acc = {0, 0, 0, 0};
    for (size_t base = (size_t)blockIdx.x * 256 * CPL; base < n16; base += (size_t)gridDim.x * 256 * CPL) {
        v4i r[CPL];
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const size_t i = base + (size_t)c * 256 + threadIdx.x;
            r[c] = __builtin_nontemporal_load(p + (i < n16 ? i : 0));
        }
#pragma unroll
        for (int c = 0; c < CPL; c++) acc ^= r[c];
    }
    if (acc.x == 0x7eadbeef && acc.y == 0x1b2c3d4e && acc.z == acc.w) sink[0] = acc.x;
}

// One wave per vector of n values: the serial sum by wave_exact_sum and by
// the chain, with the shader clocks each took (a test and timing probe).
// out[5 g ..]: fast-path sum bits, 1 if the fast path applied, chain sum
// bits, clocks of the fast path, clocks of the chain.
template <int VPL, int W>
__global__ __launch_bounds__(64 * W) void k_serial_sum_probe(const float* __restrict__ x, uint32_t n,
                                                             uint32_t* __restrict__ out) {
    __shared__ __align__(16) float e[64 * 32 + 4];
    __shared__ XsScratch<W> xs;
    const uint32_t g = blockIdx.x, tid = threadIdx.x;
    for (uint32_t i = tid; i < n; i += 64 * W) e[i] = x[(size_t)g * n + i];
    if (tid < 4) e[n + tid] = 0.0f;
    __syncthreads();
    float fast = 0.0f;
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const bool ok = block_exact_sum<VPL, W>(e, n, &xs, fast);
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    if (tid < 64) {
        const float chain = wave_chain_sum(e, n);
        const uint64_t t2 = __builtin_amdgcn_s_memtime();
        if (tid == 0) {
            out[5 * g] = __float_as_uint(fast);
            out[5 * g + 1] = ok ? 1u : 0u;
            out[5 * g + 2] = __float_as_uint(chain);
            out[5 * g + 3] = (uint32_t)(t1 - t0);
            out[5 * g + 4] = (uint32_t)(t2 - t1);
        }
    }
}

hipError_t launch_serial_sum_probe(hipStream_t st, const float* x, size_t n, size_t count, int waves,
                                   uint32_t* out) {
    if (n == 0 || n > 2048 || count == 0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)count);
#define KR_SSP(V, W) hipLaunchKernelGGL((k_serial_sum_probe<V, W>), grid, dim3(64 * W), 0, st, x, (uint32_t)n, out)
    if (waves == 1) {
        if (n <= 1024) KR_SSP(16, 1);
        else KR_SSP(32, 1);
    } else if (waves == 2) {
        if (n <= 1024) KR_SSP(8, 2);
        else KR_SSP(16, 2);
    } else if (waves == 4) {
        if (n <= 1024) KR_SSP(4, 4);
        else KR_SSP(8, 4);
    } else if (waves == 16) {
        KR_SSP(4, 16);
    } else {
        return hipErrorInvalidValue;
    }
#undef KR_SSP
    return hipGetLastError();
}

hipError_t launch_stream_read(hipStream_t st, const float* p, size_t n, int* sink, int cpl, size_t workgroups) {
    const size_t n16 = n / 4;
    if (n16 == 0) return hipSuccess;
    const size_t full = (n16 + 256 * (size_t)cpl - 1) / (256 * (size_t)cpl);
    const dim3 grid((unsigned)(workgroups == 0 ? full : std::min(workgroups, full)));
    switch (cpl) {
        case 1: hipLaunchKernelGGL(k_stream_read<1>, grid, dim3(256), 0, st, (const v4i*)p, n16, sink); break;
        case 2: hipLaunchKernelGGL(k_stream_read<2>, grid, dim3(256), 0, st, (const v4i*)p, n16, sink); break;
        case 4: hipLaunchKernelGGL(k_stream_read<4>, grid, dim3(256), 0, st, (const v4i*)p, n16, sink); break;
        case 8: hipLaunchKernelGGL(k_stream_read<8>, grid, dim3(256), 0, st, (const v4i*)p, n16, sink); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// silu (cpu.rs:708-710): x / (1 + exp(-x)), then * up.
__global__ __launch_bounds__(256) void k_silu_mul(float* __restrict__ g, const float* __restrict__ u, size_t n) {
    __shared__ uint64_t etab[32];
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const float x = i < n ? g[i] : 0.0f;
    if (threadIdx.x < 32) etab[threadIdx.x] = kExp2Tab[threadIdx.x];
    __syncthreads();
    if (i < n) {
        float s = div_rn(x, 1.0f + glibc_expf(-x, etab));
        g[i] = s * u[i];
    }
}
hipError_t launch_silu_mul(hipStream_t st, float* g, const float* u, size_t n) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, n);
    return hipGetLastError();
}

// Causal depthwise conv (cpu.rs:557-571). With `state` null, history below
// row 0 is zero padding and its terms are skipped, as conv_rows does. With a
// ring `state` (k - 1 rows, oldest first), row r reads ring row r + j where
// conv_rows would read row r - (k - 1) + j < 0, and adds that term: exactly
// what k_conv_decode computes when the rows are fed one at a time through the
// ring (cpu.rs:469-492), which is how the reference's per-token prefill of a
// Q8_0 LFM2 (lfm2.rs:490-495) sees them. The ring itself is advanced
// afterwards by k_conv_ring_advance.
__global__ void k_conv_prefill(float* __restrict__ out, const float* __restrict__ x,
                               const float* __restrict__ kern, const float* __restrict__ state, uint32_t rows,
                               uint32_t dim, uint32_t k) {
    size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (size_t)rows * dim) return;
    uint32_t r = id / dim, i = id % dim;
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; j++) {
        long h = (long)r - ((long)k - 1) + (long)j;
        if (h >= 0)
            acc += kern[(size_t)i * k + j] * x[(size_t)h * dim + i];
        else if (state)
            acc += kern[(size_t)i * k + j] * state[((size_t)r + j) * dim + i];
    }
    out[id] = acc;
}
hipError_t launch_conv_prefill(hipStream_t st, float* out, const float* x, const float* kern, size_t rows,
                               size_t dim, size_t k, const float* state) {
    size_t n = rows * dim;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_conv_prefill, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, x, kern, state,
                       (uint32_t)rows, (uint32_t)dim, (uint32_t)k);
    return hipGetLastError();
}

// The ring after `rows` rows of x have passed through it one at a time:
// ring row m holds the row at time rows - (k - 1) + m of the series
// [old ring; x]. One thread per column reads everything it needs before it
// writes, so columns never interfere.
__global__ void k_conv_ring_advance(float* __restrict__ state, const float* __restrict__ x, uint32_t rows,
                                    uint32_t dim, uint32_t k) {
    uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim) return;
    constexpr uint32_t kMaxHist = 15;
    const uint32_t hist = k - 1;
    float nv[kMaxHist];
    for (uint32_t m = 0; m < hist; m++) {
        long t = (long)rows - (long)hist + (long)m;
        nv[m] = t >= 0 ? x[(size_t)t * dim + i] : state[(size_t)((long)hist + t) * dim + i];
    }
    for (uint32_t m = 0; m < hist; m++) state[(size_t)m * dim + i] = nv[m];
}
hipError_t launch_conv_ring_advance(hipStream_t st, float* state, const float* x, size_t rows, size_t dim,
                                    size_t k) {
    if (dim == 0 || rows == 0 || k < 2) return hipSuccess;
    if (k > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_conv_ring_advance, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, st, state, x,
                       (uint32_t)rows, (uint32_t)dim, (uint32_t)k);
    return hipGetLastError();
}

// Single-row conv through the ring (cpu.rs:469-492): the output is the last
// row of the conv over [state; x], then the ring shifts by one row. All reads
// of element i happen before its writes, so `out` may alias `x`.
__global__ void k_conv_decode(float* out, const float* x, const float* __restrict__ kern, float* state,
                              uint32_t dim, uint32_t k) {
    uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim) return;
    uint32_t hist = k - 1;
    float xi = x[i];
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; j++) {
        float hv = j < hist ? state[(size_t)j * dim + i] : xi;
        acc += kern[(size_t)i * k + j] * hv;
    }
    if (hist > 0) {
        for (uint32_t j = 0; j + 1 < hist; j++) state[(size_t)j * dim + i] = state[(size_t)(j + 1) * dim + i];
        state[(size_t)(hist - 1) * dim + i] = xi;
    }
    out[i] = acc;
}
hipError_t launch_conv_decode(hipStream_t st, float* out, const float* x, const float* kern, float* state,
                              size_t dim, size_t k) {
    if (dim == 0) return hipSuccess;
    hipLaunchKernelGGL(k_conv_decode, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, st, out, x, kern, state,
                       (uint32_t)dim, (uint32_t)k);
    return hipGetLastError();
}

// The LFM2 short-conv block of one decode row (lfm2.rs:414-474) after
// in_proj: with B, C, x the three dim-wide parts of bcx, h = B * x, then the
// causal depthwise conv of h against the layer's kernel and k - 1 rows of
// state (which shifts by one, h entering last), then y = C * conv. Per
// element the same operations as k_mul, k_conv_decode and k_mul in sequence,
// in one launch.
__global__ void k_conv_block_decode(float* __restrict__ y, const float* __restrict__ bcx,
                                    const float* __restrict__ kern, float* __restrict__ state, uint32_t dim,
                                    uint32_t k) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim) return;
    const uint32_t hist = k - 1;
    const float bx = bcx[i], cx = bcx[dim + i], xx = bcx[2 * dim + i];
    const float h = bx * xx;
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; j++) {
        const float hv = j < hist ? state[(size_t)j * dim + i] : h;
        acc += kern[(size_t)i * k + j] * hv;
    }
    if (hist > 0) {
        for (uint32_t j = 0; j + 1 < hist; j++) state[(size_t)j * dim + i] = state[(size_t)(j + 1) * dim + i];
        state[(size_t)(hist - 1) * dim + i] = h;
    }
    y[i] = cx * acc;
}
hipError_t launch_conv_block_decode(hipStream_t st, float* y, const float* bcx, const float* kern, float* state,
                                    size_t dim, size_t k) {
    if (dim == 0) return hipSuccess;
    if (k < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_conv_block_decode, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, st, y, bcx, kern,
                       state, (uint32_t)dim, (uint32_t)k);
    return hipGetLastError();
}

// Embedding row (Matrix::decode_row, quant.rs:670-691): q * scale, exact.
__global__ void k_embed(const int8_t* __restrict__ q, const void* __restrict__ s, int f16, uint32_t k,
                        size_t token, const uint32_t* __restrict__ token_dev, float* __restrict__ out) {
    uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= k) return;
    size_t t = token_dev ? (size_t)token_dev[0] : token;
    size_t si = t * (k / 32) + i / 32;
    float scale = f16 ? f16w(((const uint16_t*)s)[si]) : ((const float*)s)[si];
    out[i] = (float)q[t * k + i] * scale;
}
// Many rows at once: row blockIdx.y gets the embedding of tokens[blockIdx.y].
__global__ void k_embed_rows(const int8_t* __restrict__ q, const void* __restrict__ s, int f16, uint32_t k,
                             const uint32_t* __restrict__ tokens, float* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= k) return;
    const size_t t = tokens[blockIdx.y], si = t * (k / 32) + i / 32;
    const float scale = f16 ? f16w(((const uint16_t*)s)[si]) : ((const float*)s)[si];
    out[(size_t)blockIdx.y * k + i] = (float)q[t * k + i] * scale;
}
hipError_t launch_embed_rows(hipStream_t st, const DevMatrix& e, const uint32_t* tokens_dev, size_t n, float* out) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_embed_rows, dim3((unsigned)((e.k + 255) / 256), (unsigned)n), dim3(256), 0, st, e.q, e.s,
                       e.storage == kStorageQ8_0 ? 0 : 1, (uint32_t)e.k, tokens_dev, out);
    return hipGetLastError();
}
hipError_t launch_embed(hipStream_t st, const DevMatrix& e, size_t token, const uint32_t* token_dev, float* out) {
    hipLaunchKernelGGL(k_embed, dim3((unsigned)((e.k + 255) / 256)), dim3(256), 0, st, e.q, e.s,
                       e.storage == kStorageQ8_0 ? 0 : 1, (uint32_t)e.k, token, token_dev, out);
    return hipGetLastError();
}

// argmax with Iterator::max_by(total_cmp) semantics: the largest total-order
// key wins and, among equal keys, the largest index (generate.rs:70-77).
// Each thread loads its float4s of a 16-float4-per-thread stripe at once, then
// scans them in index order; the stripes, threads and waves then reduce with
// the same tie rule. With `ring`, thread 0 also does the greedy bookkeeping:
// the token feeds the next step (out[0]), is recorded in the ring, and the
// position (out[2]) and ring index (out[5]) advance.
__device__ __forceinline__ void argmax_take(int32_t k, uint32_t i, int32_t& best, uint32_t& bi) {
    if (k > best || (k == best && i > bi)) best = k, bi = i;
}
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, uint32_t n, uint32_t* out,
                                                 uint32_t* ring, uint32_t ring_len) {
    __shared__ int32_t skey[16];
    __shared__ uint32_t sidx[16];
    constexpr uint32_t T = 1024, U = 16;
    int32_t best = INT32_MIN;
    uint32_t bi = 0;
    const uint32_t n4 = n / 4;
    for (uint32_t base = 0; base < n4; base += T * U) {
        float4 v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; u++) {
            const uint32_t f = base + u * T + threadIdx.x;
            v[u] = ((const float4*)x)[f < n4 ? f : 0];
        }
#pragma unroll
        for (uint32_t u = 0; u < U; u++) {
            const uint32_t f = base + u * T + threadIdx.x;
            if (f < n4) {
                argmax_take(total_order_key(v[u].x), 4 * f, best, bi);
                argmax_take(total_order_key(v[u].y), 4 * f + 1, best, bi);
                argmax_take(total_order_key(v[u].z), 4 * f + 2, best, bi);
                argmax_take(total_order_key(v[u].w), 4 * f + 3, best, bi);
            }
        }
    }
    for (uint32_t i = 4 * n4 + threadIdx.x; i < n; i += T) argmax_take(total_order_key(x[i]), i, best, bi);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int32_t ok = __shfl_xor(best, off);
        const uint32_t oi = __shfl_xor(bi, off);
        argmax_take(ok, oi, best, bi);
    }
    if ((threadIdx.x & 63) == 0) {
        skey[threadIdx.x >> 6] = best;
        sidx[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t b = skey[0];
        uint32_t idx = sidx[0];
        for (int w = 1; w < 16; w++) argmax_take(skey[w], sidx[w], b, idx);
        out[0] = idx;
        if (ring) {
            const uint32_t i = out[5];
            if (i < ring_len) ring[i] = idx;
            out[5] = i + 1;
            out[2] = out[2] + 1;
        }
    }
}
hipError_t launch_argmax(hipStream_t st, const float* x, size_t n, uint32_t* out) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, st, x, (uint32_t)n, out, nullptr, 0u);
    return hipGetLastError();
}

// Greedy decode: argmax into step[0] plus the ring / position bookkeeping,
// one launch.
hipError_t launch_greedy_step(hipStream_t st, const float* logits, size_t n, uint32_t* step, uint32_t* ring,
                              size_t ring_len) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, st, logits, (uint32_t)n, step, ring, (uint32_t)ring_len);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic data for benchmarks: splitmix64 per element, Box-Muller.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
    uint64_t z = splitmix64(seed ^ splitmix64(i));
    float u1 = ((float)(z >> 40) + 0.5f) * (1.0f / 16777216.0f);
    float u2 = (float)((z >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

// One thread per 32-block: draw, then quantize exactly as Q8Vec::quantize /
// Q8_0x4::from_f32 do (f32 scale for Q8_0, f16 bits for Q8_0x4, quants from
// the f32 reciprocal in both).
__global__ void k_synth_q8(int8_t* __restrict__ q, void* __restrict__ s, int f16, size_t blocks, uint64_t seed,
                           float stddev) {
    size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= blocks) return;
    float v[32];
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        v[i] = normal_at(seed, b * 32 + i) * stddev;
        amax = fmaxf(amax, fabsf(v[i]));
    }
    float d = div_rn(amax, 127.0f);
    float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
    for (int i = 0; i < 32; i++) q[b * 32 + i] = q8_round(v[i] * inv);
    if (f16)
        ((uint16_t*)s)[b] = f16_bits(d);
    else
        ((float*)s)[b] = d;
}
// Checkpoint weights to Q8 on the device: Matrix::from_f32_q8_0 (Q8Vec::quantize,
// quant.rs:544-557, 856-874) and Q8_0x4::from_f32 (quant.rs:124-164) for rows
// [row0, row0 + rows) of a matrix, from f32 values or from bf16 bits widened
// exactly (bits << 16, hf.rs widen). One half-wave per 32-block, as k_quantize:
// coalesced loads, the block amax by an order-free max reduction, then every
// lane rounds its own element with the f32 reciprocal; Q8_0 keeps the f32 scale,
// Q8_0x4 its f16 bits.
template <bool BF16>
__global__ __launch_bounds__(256) void k_quant_weights(const void* __restrict__ src, size_t blocks,
                                                      int8_t* __restrict__ q, void* __restrict__ s, int f16) {
    const size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t blk = gid >> 5;
    const int lane = threadIdx.x & 31;
    const bool valid = blk < blocks;
    const size_t e = valid ? blk * 32 + lane : 0;
    const float v = BF16 ? u2f((uint32_t)((const uint16_t*)src)[e] << 16) : ((const float*)src)[e];
    float m = fmaxf(0.0f, fabsf(v));
    m = group_max32(m);
    const float d = div_rn(m, 127.0f);
    const float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
    if (valid) {
        q[e] = q8_round(v * inv);
        if (lane == 0) {
            if (f16)
                ((uint16_t*)s)[blk] = f16_bits(d);
            else
                ((float*)s)[blk] = d;
        }
    }
}
hipError_t launch_quant_weights(hipStream_t st, const DevMatrix& m, size_t row0, size_t rows, const void* src,
                                int bf16) {
    const size_t nb = m.k / 32, blocks = rows * nb;
    if (blocks == 0) return hipSuccess;
    int8_t* q = m.q + row0 * m.k;
    const int f16 = m.storage == kStorageQ8_0 ? 0 : 1;
    void* s = f16 ? (void*)((uint16_t*)m.s + row0 * nb) : (void*)((float*)m.s + row0 * nb);
    const dim3 grid((unsigned)((blocks * 32 + 255) / 256));
    if (bf16)
        hipLaunchKernelGGL(k_quant_weights<true>, grid, dim3(256), 0, st, src, blocks, q, s, f16);
    else
        hipLaunchKernelGGL(k_quant_weights<false>, grid, dim3(256), 0, st, src, blocks, q, s, f16);
    return hipGetLastError();
}

hipError_t launch_synthetic_q8(hipStream_t st, const DevMatrix& m, uint64_t seed, float stddev) {
    size_t blocks = m.n * m.k / 32;
    hipLaunchKernelGGL(k_synth_q8, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, st, m.q, m.s,
                       m.storage == kStorageQ8_0 ? 0 : 1, blocks, seed, stddev);
    return hipGetLastError();
}

// int8 MFMA throughput probe for benchmarks: every wave keeps four
// independent accumulators in flight through `iters` rounds of the int8 MFMA
// of the kind asked (0: 32x32x32, 1: 16x16x32, the one the Q8_0 GEMM uses);
// the sums go to `sink` so the work is not removed.
template <int KIND>
__global__ __launch_bounds__(256) void k_mfma_spin(int* __restrict__ sink, uint32_t iters) {
    const int t = (int)threadIdx.x;
    int s = 0;
    if (KIND == 0) {
        const v4i a = {t, t + 1, t + 2, t + 3}, b = {3 * t, t ^ 5, t + 7, 1};
        v16i acc[4] = {};
        for (uint32_t i = 0; i < iters; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
#pragma unroll
        for (int c = 0; c < 4; c++) s += acc[c][c];
    } else {
        const long a = (long)t * 0x0101010101LL, b = (long)(t ^ 3) * 0x0303030303LL;
        v4i acc[4] = {};
        for (uint32_t i = 0; i < iters; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, acc[c], 0, 0, 0);
#pragma unroll
        for (int c = 0; c < 4; c++) s += acc[c][c];
    }
    sink[(size_t)blockIdx.x * blockDim.x + t] = s;
}
hipError_t launch_mfma_spin(hipStream_t st, int kind, int* sink, size_t blocks, uint32_t iters, double* ops) {
    const double per = kind == 0 ? 2.0 * 32 * 32 * 32 : 2.0 * 16 * 16 * 32;  // int8 ops per instruction
    *ops = per * 4 * iters * 4 * (double)blocks;  // 4 per round x 4 waves per workgroup
    if (kind == 0)
        hipLaunchKernelGGL(k_mfma_spin<0>, dim3((unsigned)blocks), dim3(256), 0, st, sink, iters);
    else
        hipLaunchKernelGGL(k_mfma_spin<1>, dim3((unsigned)blocks), dim3(256), 0, st, sink, iters);
    return hipGetLastError();
}

// The f32 values k_synth_q8 quantizes (element i of the flattened matrix).
__global__ void k_synth_values(float* __restrict__ out, size_t n, uint64_t seed, float stddev) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = normal_at(seed, i) * stddev;
}
hipError_t launch_synthetic_values(hipStream_t st, float* out, size_t n, uint64_t seed, float stddev) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_synth_values, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, seed, stddev);
    return hipGetLastError();
}

__global__ void k_synth_normal(float* __restrict__ out, size_t n, uint64_t seed) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = normal_at(seed, i);
}
hipError_t launch_synthetic_normal(hipStream_t st, float* out, size_t n, uint64_t seed) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_synth_normal, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, seed);
    return hipGetLastError();
}

// x86 logits over a Q8_0x4 classifier re-quantize each decoded row
// (quant.rs:232-235). With every block's max |q| in {0, 127} that gives back
// the stored quants and the widened f16 scale; count the blocks where not.
__global__ void k_requant_check(const int8_t* __restrict__ q, size_t blocks, unsigned int* counter) {
    size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= blocks) return;
    int m = 0;
    for (int i = 0; i < 32; i++) {
        int a = q[b * 32 + i];
        a = a < 0 ? -a : a;
        m = a > m ? a : m;
    }
    if (m != 0 && m != 127) atomicAdd(counter, 1u);
}
hipError_t launch_requant_check(hipStream_t st, const DevMatrix& m, unsigned int* counter) {
    size_t blocks = m.n * m.k / 32;
    hipLaunchKernelGGL(k_requant_check, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, st, m.q, blocks,
                       counter);
    return hipGetLastError();
}

// The literal re-quantization, for classifiers where the identity fails.
__global__ void k_requantize(const int8_t* __restrict__ q, const uint16_t* __restrict__ s, int8_t* __restrict__ q2,
                             float* __restrict__ s2, size_t blocks) {
    size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= blocks) return;
    float sc = f16w(s[b]);
    float v[32];
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        v[i] = (float)q[b * 32 + i] * sc;
        amax = fmaxf(amax, fabsf(v[i]));
    }
    float d = div_rn(amax, 127.0f);
    float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
    for (int i = 0; i < 32; i++) q2[b * 32 + i] = q8_round(v[i] * inv);
    s2[b] = d;
}
hipError_t launch_requantize(hipStream_t st, const DevMatrix& src, const DevMatrix& dst) {
    size_t blocks = src.n * src.k / 32;
    hipLaunchKernelGGL(k_requantize, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, st, src.q,
                       (const uint16_t*)src.s, dst.q, (float*)dst.s, blocks);
    return hipGetLastError();
}

}  // namespace kr

// Prefill attention on the matrix core (k_attn_mx_*). Built as its own
// translation unit with -mllvm -amdgpu-mfma-vgpr-form=1, so that the f32
// MFMA results land in ordinary vector registers: the vector unit adds them
// to its chains without a register-file move per value.
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "kernels.hpp"
#include "numerics.hpp"

namespace kr {

typedef float mx_v32f __attribute__((ext_vector_type(32)));
// Attention of prefill rows on the matrix core, in three launches over
// blocks of 32 (row, head) pairs (G query heads of one KV head x 32 / G
// rows whose windows share a layout). f32 MFMA with one nonzero product per
// output is an exact fused multiply-add (every output of
// v_mfma_f32_32x32x1_2b_f32 with a zero or accumulating C is fmaf(a, b, c),
// subnormals and cancellation included), so the reference's chains run on
// it unchanged:
//  1. k_attn_mx_scores: per 32-position tile, the four FMA chains of the dot
//     (dot.rs:360) over 32 pairs x 32 positions, two chains per instruction
//     (blocks 0 and 1 = chains 0 and 2, then 1 and 3; lane l of half h
//     brings dims 4s + 2h and 4s + 2h + 1 of its pair's q and of its
//     position's key), then ((a0 + a1) + (a2 + a3)) * scale (cpu.rs:609) on
//     the vector unit. Raw scores go to `att`.
//  2. k_attn_softmax_att (elementwise.rs:65-91): with each pair's max from
//     the scores launch, the exps back to `att` and each pair's serial sum,
//     64 pairs per workgroup over 64-position chunks.
//  3. k_attn_mx_v: each exp divided by its pair's sum as the chunk is staged
//     (the probabilities back to `att` where the caller keeps them, as the
//     reference leaves them); per two positions one instruction forms the 32 pairs x
//     32 dims products p_i * v_i[e] (each the correctly rounded product), and
//     the vector unit adds them to the chains in position order. Positions a
//     pair's window does not reach get p = 0; the zero products leave the
//     sums unchanged (the sums start at +0 and never become -0). A block
//     whose V rows past its shortest window hold an infinity or NaN (0 * inf
//     is NaN) recomputes its sums over each pair's own window instead.
struct MxBlock {
    uint32_t r0, nr, h0, kvo, n_shared, cmax;
    DevWindow w0;
};
template <int G>
__device__ __forceinline__ MxBlock mx_block(const DevWindow* windows, uint32_t n_rows, uint32_t kv_mul, uint32_t hs,
                                            uint32_t* s_cnt) {
    constexpr uint32_t R = 32 / G;
    MxBlock b;
    // the last row blocks first: a causal prefill's windows grow with the
    // row, so the longest blocks start first and the short ones fill in
    // behind them, instead of leaving the long ones for the tail
    b.r0 = (gridDim.y - 1 - blockIdx.y) * R;
    b.nr = min(R, n_rows - b.r0);
    b.h0 = blockIdx.x * G;
    b.kvo = (b.h0 / kv_mul) * hs;
    b.w0 = windows[b.r0];
    b.n_shared = b.w0.shared_end - b.w0.shared_start;
    if (threadIdx.x < 32) {
        const uint32_t r = threadIdx.x / G;
        s_cnt[threadIdx.x] = r < b.nr ? b.n_shared + windows[b.r0 + r].slot - b.w0.att_start + 1 : 0;
    }
    __syncthreads();
    b.cmax = 0;
    for (uint32_t k = 0; k < 32; k++) b.cmax = max(b.cmax, s_cnt[k]);
    return b;
}

template <int G, int HS>
__global__ __launch_bounds__(256) void k_attn_mx_scores(const float* __restrict__ q, float* __restrict__ att,
                                                        const float* __restrict__ kc, size_t loff,
                                                        const DevWindow* __restrict__ windows, uint32_t n_rows,
                                                        uint32_t n_heads, uint32_t kv_mul, uint32_t kv_dim,
                                                        uint32_t seq_len, float scale, float* __restrict__ pmax) {
    constexpr uint32_t NS = HS / 4, KCH = 8, QST = HS + 4;
    static_assert(32 % G == 0 && (HS == 64 || HS == 128) && NS % KCH == 0, "shape");
    __shared__ __align__(16) float s_q[32 * QST];  // the pairs' q rows
    // each wave's key chunk: [32 positions][KCH steps x 4 dims], rows padded to
    // KST floats so that the lane-per-position float2 reads meet distinct banks
    constexpr uint32_t KST = 4 * KCH + 2;
    __shared__ __align__(16) float s_k[4][32 * KST];
    __shared__ uint32_t s_cnt[32];
    __shared__ float s_mx[4][32];
    const uint32_t tid = threadIdx.x, lane = tid & 63, h = lane >> 5, pr = lane & 31;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t width = n_heads * HS;
    const MxBlock B = mx_block<G>(windows, n_rows, kv_mul, HS, s_cnt);
    const uint32_t r0 = B.r0, nr = B.nr, h0 = B.h0, n_shared = B.n_shared, cmax = B.cmax;
    const DevWindow w0 = B.w0;
    // q rows of the 32 pairs (pairs past the block read the last one)
    for (uint32_t f = tid; f < 32 * (HS / 4); f += 256) {
        const uint32_t pair = f / (HS / 4), col = f - pair * (HS / 4);
        const uint32_t qp = min(pair, nr * G - 1), qr = qp / G, qj = qp - qr * G;
        *(float4*)(s_q + pair * QST + 4 * col) =
            *(const float4*)(q + (size_t)(r0 + qr) * width + (size_t)(h0 + qj) * HS + 4 * col);
    }
    __syncthreads();
    const float* kbase = kc + loff + B.kvo;
    auto att_row = [&](uint32_t pair) {
        const uint32_t r = pair / G, j = pair - r * G;
        return att + (size_t)(r0 + r) * n_heads * seq_len + (size_t)(h0 + j) * seq_len;
    };
    // 1. scores
    {
        // this lane's pair's q dims 4s + 2h, 4s + 2h + 1, from LDS
        const float* qrow = s_q + pr * QST + 2 * h;
        const uint32_t ntile = (cmax + 31) / 32;
        // this wave's tiles t = wave, wave + 4, ...; key chunks of KCH steps
        // (32 positions x 4 KCH dims) read with 4 KCH / 4 lanes on each
        // position's contiguous 16 KCH bytes (a lane per position reading its
        // own 8 bytes per step would spread every load over 32 rows), through
        // two register sets used in turn, the next chunk (the next tile's
        // first at a tile's end) in flight while one is used; each chunk goes
        // through the wave's LDS rows to the lane of its position
        constexpr uint32_t NCH = NS / KCH, SEG = KCH, RPL = 64 / SEG, NLD = 32 / RPL;
        static_assert(NCH % 2 == 0 && 64 % SEG == 0, "a tile starts in the first register set");
        typedef float kv4 __attribute__((ext_vector_type(4)));
        const uint32_t lrow = lane / SEG, lseg = lane - lrow * SEG;
        auto kload = [&](kv4(&k)[NLD], uint32_t t, uint32_t c) {
#pragma unroll
            for (uint32_t i = 0; i < NLD; i++) {
                const uint32_t pos = min(32 * t + RPL * i + lrow, cmax - 1);
                k[i] = *(const kv4*)(kbase + (size_t)win_slot(w0, n_shared, pos) * kv_dim + 4 * (c * KCH + lseg));
            }
        };
        float* kt = s_k[wave];
        auto kput = [&](const kv4(&k)[NLD]) {
#pragma unroll
            for (uint32_t i = 0; i < NLD; i++) {
                float* d = kt + (RPL * i + lrow) * KST + 4 * lseg;
                *(float2*)d = float2{k[i].x, k[i].y};
                *(float2*)(d + 2) = float2{k[i].z, k[i].w};
            }
            __builtin_amdgcn_wave_barrier();  // one wave's LDS accesses complete in order
        };
        float mloc[16];  // the max of element v's pair over this lane's positions (order-free)
#pragma unroll
        for (uint32_t v = 0; v < 16; v++) mloc[v] = -INFINITY;
        kv4 ka[NLD], kb[NLD];
        if (wave < ntile) kload(ka, wave, 0);
        for (uint32_t t = wave; t < ntile; t += 4) {
            const uint32_t tnext = min(t + 4, ntile - 1);
            mx_v32f a02 = {}, a13 = {};
            auto steps = [&](uint32_t c) {
                // this lane's position pr, dims 4 (c KCH + u) + 2 h and + 1
                float2 k[KCH];
#pragma unroll
                for (uint32_t u = 0; u < KCH; u++) k[u] = *(const float2*)(kt + pr * KST + 4 * u + 2 * h);
                __builtin_amdgcn_wave_barrier();  // the reads come before the next chunk's stores
#pragma unroll
                for (uint32_t u = 0; u < KCH; u++) {
                    const float2 qq = *(const float2*)(qrow + 4 * (c * KCH + u));
                    a02 = __builtin_amdgcn_mfma_f32_32x32x1f32(qq.x, k[u].x, a02, 0, 0, 0);
                    a13 = __builtin_amdgcn_mfma_f32_32x32x1f32(qq.y, k[u].y, a13, 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);  // no chunk's q reads move above the previous chunk
            };
#pragma unroll
            for (uint32_t c = 0; c < NCH; c += 2) {
                kload(kb, t, c + 1);
                kput(ka);
                steps(c);
                if (c + 2 < NCH)
                    kload(ka, t, c + 2);
                else
                    kload(ka, tnext, 0);  // the next tile's first chunk (the last tile's again at the end)
                kput(kb);
                steps(c + 1);
            }
            // element v: pair 8 (v / 4) + 4 h + v % 4, position 32 t + pr; a02 = chains 0 | 2, a13 = 1 | 3
            const uint32_t pos = 32 * t + pr;
#pragma unroll
            for (uint32_t v = 0; v < 16; v++) {
                const uint32_t pair = 8 * (v >> 2) + 4 * h + (v & 3);
                const float sv = ((a02[v] + a13[v]) + (a02[16 + v] + a13[16 + v])) * scale;
                if (pos < s_cnt[pair]) {
                    att_row(pair)[pos] = sv;
                    mloc[v] = fmaxf(mloc[v], sv);
                }
            }
        }
        // each pair's max (NaN ignored, as f32::max): over the 32 positions of a
        // half-wave, then over the waves
#pragma unroll
        for (uint32_t v = 0; v < 16; v++) {
            const float mv = group_max32(mloc[v]);
            if (pr == 0) s_mx[wave][8 * (v >> 2) + 4 * h + (v & 3)] = mv;
        }
    }
    __syncthreads();
    if (tid < 32 && s_cnt[tid] > 0) {
        const uint32_t r = tid / G, j = tid - r * G;
        pmax[(size_t)(r0 + r) * n_heads + h0 + j] =
            fmaxf(fmaxf(s_mx[0][tid], s_mx[1][tid]), fmaxf(s_mx[2][tid], s_mx[3][tid]));
    }
}

// Exps and sums of the softmax of kMxSmPairs (row, head) pairs of `att`
// per workgroup (elementwise.rs:65-91), over 64-position chunks; wave w
// serves pairs PW w .. + PW - 1, one pair per load (lane = position: 256
// contiguous bytes). With each pair's max from k_attn_mx_scores, the exps go
// to `att` and to the wave's rows of an LDS tile [pair][position], and lane
// k < PW runs pair PW w + k's serial sum over its row in position order. The
// division by the sum happens where the probabilities are next read
// (k_attn_mx_v). A wave's time is PW times its pairs' longest window in
// exps, and the waves of the longest windows set the launch's length: with
// 4 pairs a wave they do a quarter of the work they did with 16 (cfg5
// 2048-token prefill 106.8k -> 113.6k tok/s at 8 pairs, 116.7k at 4;
// 2 and 1 are slower again, the serial sums then dominating).
static constexpr uint32_t kMxSmPW = 4, kMxSmPairs = 4 * kMxSmPW;
__global__ __launch_bounds__(256) void k_attn_softmax_att(float* __restrict__ att,
                                                          const DevWindow* __restrict__ windows, uint32_t n_rows,
                                                          uint32_t n_heads, uint32_t seq_len,
                                                          const float* __restrict__ pmax, float* __restrict__ psum) {
    // chunk positions, tile row stride (16-byte rows, each 16 bytes further
    // along the banks than the one above), pairs per wave
    constexpr uint32_t C = 64, TS = C + 4, PW = kMxSmPW, PP = kMxSmPairs;
    __shared__ __align__(16) float s_e[PP * TS];
    __shared__ uint64_t etab[32];
    __shared__ uint32_t s_n[PP];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the last pairs first (the longest windows of a causal prefill; see mx_block)
    const uint32_t n_pairs = n_rows * n_heads, p0 = (gridDim.x - 1 - blockIdx.x) * PP;
    if (tid < 32) etab[tid] = kExp2Tab[tid];
    if (tid < PP) {
        uint32_t n = 0;
        if (p0 + tid < n_pairs) {
            const DevWindow w = windows[(p0 + tid) / n_heads];
            n = w.shared_end - w.shared_start + w.slot - w.att_start + 1;
        }
        s_n[tid] = n;
    }
    __syncthreads();
    uint32_t nmax = 0;
    for (uint32_t k = 0; k < PP; k++) nmax = max(nmax, s_n[k]);
    const uint32_t nch = (nmax + C - 1) / C;
    auto pidx = [&](uint32_t k) { return min(p0 + PW * wave + k, n_pairs - 1); };
    auto row = [&](uint32_t k) { return att + (size_t)pidx(k) * seq_len; };
    // every load is unconditional, at a position inside the longest window
    // (values past a pair's own window are selected away, never used), so
    // the loads of a batch are all in flight together
    auto at = [&](uint32_t i) { return i < nmax ? i : nmax - 1; };
    float m[PW];
#pragma unroll
    for (uint32_t k = 0; k < PW; k++) m[k] = pmax[pidx(k)];
    float sum = 0.0f;
    float* tw = s_e + PW * wave * TS;
    // chunk c + 1's loads are issued before chunk c's exps and chains run
    // (two register sets in turn; a load past the last chunk re-reads a
    // position inside the window and is not used)
    auto load = [&](float (&x)[PW], uint32_t c) {
        const uint32_t i = c * C + lane;
#pragma unroll
        for (uint32_t k = 0; k < PW; k++) x[k] = row(k)[at(i)];
    };
    auto process = [&](const float (&x)[PW], uint32_t c) {
        const uint32_t i = c * C + lane;
#pragma unroll
        for (uint32_t k = 0; k < PW; k++) {
            const bool live = i < s_n[PW * wave + k];
            const float ev = live ? glibc_expf(x[k] - m[k], etab) : 0.0f;
            if (live) row(k)[i] = ev;
            tw[k * TS + lane] = ev;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's tile stores have landed
        __builtin_amdgcn_wave_barrier();
        if (lane < PW) {  // past a window's end: +0.0, which leaves the sum unchanged
            const float4* r = (const float4*)(tw + lane * TS);
#pragma unroll
            for (uint32_t k = 0; k < C / 4; k++) {
                const float4 f = r[k];
                sum += f.x;
                sum += f.y;
                sum += f.z;
                sum += f.w;
            }
        }
        __builtin_amdgcn_wave_barrier();  // the chains have read the tile before it is rewritten
    };
    float xa[PW], xb[PW];
    load(xa, 0);
    uint32_t c = 0;
    for (; c + 2 <= nch; c += 2) {
        load(xb, c + 1);
        process(xa, c);
        load(xa, c + 2);
        process(xb, c + 1);
    }
    if (c < nch) process(xa, c);
    if (lane < PW && p0 + PW * wave + lane < n_pairs) psum[p0 + PW * wave + lane] = sum;
}

template <int G, int HS>
__global__ __launch_bounds__(256, 3) void k_attn_mx_v(float* __restrict__ att, float* __restrict__ out,
                                                   const float* __restrict__ vc, size_t loff,
                                                   const DevWindow* __restrict__ windows, uint32_t n_rows,
                                                   uint32_t n_heads, uint32_t kv_mul, uint32_t kv_dim,
                                                   uint32_t seq_len, int8_t* __restrict__ qo, float* __restrict__ so,
                                                   uint16_t* __restrict__ ho, const float* __restrict__ psum,
                                                   uint32_t keep_att) {
    constexpr uint32_t VST = HS + 4, PST = 33;
    static_assert(32 % G == 0 && (HS == 64 || HS == 128), "shape");
    __shared__ __align__(16) float s_v[2][32 * VST];  // V chunk [position][dim]
    __shared__ float s_p[2][32 * PST];                // probability chunk [position][pair]
    __shared__ uint32_t s_cnt[32];
    const uint32_t tid = threadIdx.x, lane = tid & 63, h = lane >> 5, pr = lane & 31;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t width = n_heads * HS;
    const MxBlock B = mx_block<G>(windows, n_rows, kv_mul, HS, s_cnt);
    const uint32_t r0 = B.r0, nr = B.nr, h0 = B.h0, n_shared = B.n_shared, cmax = B.cmax;
    const DevWindow w0 = B.w0;
    const float* vbase = vc + loff + B.kvo;
    auto att_row = [&](uint32_t pair) {
        const uint32_t r = pair / G, j = pair - r * G;
        return att + (size_t)(r0 + r) * n_heads * seq_len + (size_t)(h0 + j) * seq_len;
    };
    // Positions past a pair's window enter its sums as p = 0 times v, which
    // is 0 only for a finite v. The shortest live window: V rows from there
    // on are checked as they are staged, and a block that met an infinite or
    // NaN one recomputes its sums under each pair's own window at the end.
    uint32_t cmin = cmax;
    for (uint32_t k = 0; k < nr * G; k++) cmin = min(cmin, s_cnt[k]);
    cmin = __builtin_amdgcn_readfirstlane(cmin);
    bool vbad = false;
    // 3. V sums: wave w owns dims 32 w .. 32 w + 31 (HS / 32 waves); chunks
    // of 32 positions staged through LDS, the next chunk's loads in flight
    typedef float vs4 __attribute__((ext_vector_type(4)));  // native vectors: the stages stay in registers
    struct VStage {
        vs4 v[HS / 32];
        vs4 p;
    };
    const uint32_t nch = (cmax + 31) / 32;
    // loader: V piece f = tid + 256 k (position f / (HS/4), float4 f % (HS/4)); probabilities: pair tid / 8,
    // positions 4 (tid % 8) .. + 3
    auto gload = [&](VStage& st, uint32_t c) {
        c = c < nch ? c : nch - 1;
#pragma unroll
        for (uint32_t k = 0; k < HS / 32; k++) {
            const uint32_t f = tid + 256 * k, rr = f / (HS / 4), col = f - rr * (HS / 4);
            st.v[k] = *(const vs4*)(vbase + (size_t)win_slot(w0, n_shared, min(32 * c + rr, cmax - 1)) * kv_dim + 4 * col);
        }
        const uint32_t pair = tid >> 3, i0 = 32 * c + 4 * (tid & 7), n = s_cnt[pair];
        const float* row = att_row(min(pair, nr * G - 1));
        // loads inside the longest window (always), values past the pair's own set to 0
        const uint32_t lim = cmax - 1;
        const float p0 = row[min(i0, lim)], p1 = row[min(i0 + 1, lim)], p2 = row[min(i0 + 2, lim)],
                    p3 = row[min(i0 + 3, lim)];
        st.p = vs4{i0 < n ? p0 : 0.0f, i0 + 1 < n ? p1 : 0.0f, i0 + 2 < n ? p2 : 0.0f, i0 + 3 < n ? p3 : 0.0f};
    };
    // the probabilities: each exp divided by its pair's sum (elementwise.rs:88-91),
    // written back to `att` where the reference leaves them (unless the
    // caller has no use for them: keep_att == 0), and to LDS
    const uint32_t lpair = tid >> 3, lr = lpair / G, lj = lpair - lr * G;
    const float lsum = s_cnt[lpair] > 0 ? psum[(size_t)(r0 + lr) * n_heads + h0 + lj] : 1.0f;
    uint32_t lchunk = 0;  // the chunk lstore is given next
    auto lstore = [&](VStage& st, int buf) {
        const uint32_t g0 = 32 * lchunk++ + 4 * (tid & 7), n = s_cnt[lpair];
        float* arow = att_row(min(lpair, nr * G - 1));
        if (g0 < n) st.p.x = div_rn(st.p.x, lsum);
        if (g0 + 1 < n) st.p.y = div_rn(st.p.y, lsum);
        if (g0 + 2 < n) st.p.z = div_rn(st.p.z, lsum);
        if (g0 + 3 < n) st.p.w = div_rn(st.p.w, lsum);
        if (keep_att) {
            if (g0 < n) arow[g0] = st.p.x;
            if (g0 + 1 < n) arow[g0 + 1] = st.p.y;
            if (g0 + 2 < n) arow[g0 + 2] = st.p.z;
            if (g0 + 3 < n) arow[g0 + 3] = st.p.w;
        }
#pragma unroll
        for (uint32_t k = 0; k < HS / 32; k++) {
            const uint32_t f = tid + 256 * k, rr = f / (HS / 4), col = f - rr * (HS / 4);
            *(vs4*)(s_v[buf] + rr * VST + 4 * col) = st.v[k];
        }
        if (32 * lchunk > cmin) {  // this chunk reaches past the shortest window
#pragma unroll
            for (uint32_t k = 0; k < HS / 32; k++) {
                const uint32_t rr = (tid + 256 * k) / (HS / 4);
                const vs4 x = st.v[k];
                if (32 * (lchunk - 1) + rr >= cmin && !(__builtin_isfinite(x.x) && __builtin_isfinite(x.y) &&
                                                        __builtin_isfinite(x.z) && __builtin_isfinite(x.w)))
                    vbad = true;
            }
        }
        const uint32_t pair = tid >> 3, i0 = 4 * (tid & 7);
        s_p[buf][i0 * PST + pair] = st.p.x;
        s_p[buf][(i0 + 1) * PST + pair] = st.p.y;
        s_p[buf][(i0 + 2) * PST + pair] = st.p.z;
        s_p[buf][(i0 + 3) * PST + pair] = st.p.w;
    };
    float o[16];
#pragma unroll
    for (uint32_t v = 0; v < 16; v++) o[v] = 0.0f;
    const bool vwave = wave < HS / 32;
    const uint32_t d0 = 32 * (vwave ? wave : 0);
    auto compute = [&](int buf, uint32_t c) {
        if (c >= nch || !vwave) return;
        const float* pb = s_p[buf] + h * PST + pr;
        const float* vb = s_v[buf] + h * VST + d0 + pr;
        // the next step's instruction is issued before this step's adds, its
        // operands read two steps ahead, so neither waits on the other
        float pa[16], va[16];
        // operands a quarter at a time, each issued a quarter ahead of its use
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) pa[k] = pb[2 * k * PST], va[k] = vb[2 * k * VST];
        mx_v32f d = __builtin_amdgcn_mfma_f32_32x32x1f32(pa[0], va[0], mx_v32f{}, 0, 0, 0);
#pragma unroll
        for (uint32_t k = 0; k < 16; k++) {
            if (k % 4 == 0 && k + 8 < 16) {
#pragma unroll
                for (uint32_t q = k + 8; q < k + 12; q++) pa[q] = pb[2 * q * PST], va[q] = vb[2 * q * VST];
            }
            mx_v32f dn;
            if (k + 1 < 16) dn = __builtin_amdgcn_mfma_f32_32x32x1f32(pa[k + 1], va[k + 1], mx_v32f{}, 0, 0, 0);
#pragma unroll
            for (uint32_t v = 0; v < 16; v++) o[v] += d[v];  // position 2 k
#pragma unroll
            for (uint32_t v = 0; v < 16; v++) o[v] += d[16 + v];  // position 2 k + 1
            if (k + 1 < 16) d = dn;
        }
    };
    // one register stage: chunk c + 1 is in flight while chunk c is
    // computed from LDS (a second stage, chunk c + 2 in flight, cost 13
    // spilled registers at three waves per SIMD and ran 1.2% slower)
    VStage sa;
    gload(sa, 0);
    lstore(sa, 0);
    gload(sa, 1);
    __syncthreads();
    for (uint32_t c = 0; c < nch; c += 2) {
        compute(0, c);
        lstore(sa, 1);  // chunk c + 1
        gload(sa, c + 2);
        __syncthreads();
        compute(1, c + 1);
        lstore(sa, 0);  // chunk c + 2
        gload(sa, c + 3);
        __syncthreads();
    }
    if (__syncthreads_or(vbad) && vwave) {
        // the reference's loop for each element, in position order, over its
        // own window only: the probabilities from `att`, V from the cache
#pragma unroll
        for (uint32_t v = 0; v < 16; v++) {
            const uint32_t pair = 8 * (v >> 2) + 4 * h + (v & 3);
            const uint32_t n = pair < nr * G ? s_cnt[pair] : 0;
            const float* prow = att_row(min(pair, nr * G - 1));
            float acc = 0.0f;
            for (uint32_t i = 0; i < n; i++)
                acc += prow[i] * vbase[(size_t)win_slot(w0, n_shared, i) * kv_dim + d0 + pr];
            o[v] = acc;
        }
    }
    if (!vwave) return;
    // element v: pair 8 (v / 4) + 4 h + v % 4, dim d0 + pr
#pragma unroll
    for (uint32_t v = 0; v < 16; v++) {
        const uint32_t pair = 8 * (v >> 2) + 4 * h + (v & 3), r = pair / G, j = pair - r * G;
        const bool live = r < nr;
        const size_t oi = (size_t)(r0 + r) * width + (size_t)(h0 + j) * HS + d0 + pr;
        if (live) out[oi] = o[v];
        if (qo) quant_lane(o[v], live, qo + oi, so + oi / 32, ho + oi / 32);  // quant.rs:864-873
    }
}

// the shortest longest-window the matrix-core launches take: for head_dim
// 128 they overtake k_attn_rows between 128 and 192 positions (cfg5 prefill
// of 128 tokens 54.6k against 50.5k tok/s, of 192 tokens 59.5k against 61.7k,
// of 1000 tokens 69k against 125k); for head_dim 64 k_attn_rows stages its
// keys through LDS and stays faster up to about 768 (1.7B-shaped prefills:
// 256 / 640 tokens 65.1k / 71.0k on k_attn_rows against 57.6k / 69.7k, 768
// even, 896 / 1000 tokens 74.9k / 72.0k against 78.1k / 78.4k)
static constexpr size_t kAttnMxMinWindow128 = 160, kAttnMxMinWindow64 = 768;
// the launches loop over the window in chunks, so the longest window is a
// choice, not a limit of the kernels (k_attn_rows and k_attention_fast, which
// took the windows past 4096 before, ran 2048 -> 4200-token prefills at a
// third of the rate)
static constexpr size_t kAttnMxMaxWindow = 16384;
// k_attn_mx: query heads per workgroup (the largest of 8, 4, 2, 1 dividing
// kv_mul), and whether a launch can take it: head size 64 or 128, windows
// of at most kAttnMxMaxWindow positions, n_rows >= 2 and every block of 32 / G rows
// sharing one window layout (prefill).
static size_t attn_mx_group(size_t kv_mul) {
    for (size_t g : {8, 4, 2})
        if (kv_mul % g == 0) return g;
    return 1;
}
bool attention_mx_ok(const DevWindow* w, size_t n_rows, size_t max_count, size_t kv_mul, size_t hs) {
    // shorter windows run faster on k_attn_rows (one launch, more workgroups)
    const size_t min_window = hs == 128 ? kAttnMxMinWindow128 : kAttnMxMinWindow64;
    if ((hs != 64 && hs != 128) || max_count < min_window || max_count > kAttnMxMaxWindow || n_rows < 2) return false;
    const size_t R = 32 / attn_mx_group(kv_mul);
    for (size_t r = 0; r < n_rows; r++) {
        const DevWindow& a = w[r - r % R];
        if (a.att_start != w[r].att_start || a.shared_start != w[r].shared_start || a.shared_end != w[r].shared_end)
            return false;
    }
    return true;
}

hipError_t launch_attention_mx(hipStream_t st, const float* q, float* out, float* att, const float* kc,
                               const float* vc, size_t layer, const DevWindow* windows, size_t n_rows,
                               size_t max_count, size_t n_heads, size_t kv_mul, size_t hs, size_t kv_dim,
                               size_t seq_len, float scale, int8_t* qo, float* so, uint16_t* ho, float* scratch,
                               bool keep_att) {
    const size_t G = attn_mx_group(kv_mul), R = 32 / G;
    const dim3 grid((unsigned)(n_heads / G), (unsigned)((n_rows + R - 1) / R));
    const dim3 gsm((unsigned)((n_rows * n_heads + kMxSmPairs - 1) / kMxSmPairs));
    float* pmax = scratch;                  // each pair's max
    float* psum = scratch + n_rows * n_heads;  // and its sum of exps
#define KR_ATTN_MX(g, h)                                                                                         \
    hipLaunchKernelGGL((k_attn_mx_scores<g, h>), grid, dim3(256), 0, st, q, att, kc, layer * seq_len * kv_dim,      \
                       windows, (uint32_t)n_rows, (uint32_t)n_heads, (uint32_t)kv_mul, (uint32_t)kv_dim,           \
                       (uint32_t)seq_len, scale, pmax);                                                            \
    hipLaunchKernelGGL(k_attn_softmax_att, gsm, dim3(256), 0, st, att, windows, (uint32_t)n_rows, (uint32_t)n_heads, \
                       (uint32_t)seq_len, pmax, psum);                                                             \
    hipLaunchKernelGGL((k_attn_mx_v<g, h>), grid, dim3(256), 0, st, att, out, vc, layer * seq_len * kv_dim, windows, \
                       (uint32_t)n_rows, (uint32_t)n_heads, (uint32_t)kv_mul, (uint32_t)kv_dim, (uint32_t)seq_len, \
                       qo, so, ho, psum, keep_att ? 1u : 0u)
#define KR_ATTN_MX_G(g)     \
    if (hs == 64) {         \
        KR_ATTN_MX(g, 64);  \
    } else {                \
        KR_ATTN_MX(g, 128); \
    }
    switch (G) {
        case 8: KR_ATTN_MX_G(8) break;
        case 4: KR_ATTN_MX_G(4) break;
        case 2: KR_ATTN_MX_G(2) break;
        default: KR_ATTN_MX_G(1) break;
    }
#undef KR_ATTN_MX_G
#undef KR_ATTN_MX
    return hipGetLastError();
}

}  // namespace kr

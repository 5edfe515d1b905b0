// Q8_0 GEMM with the reference's four partial sums (dot.rs:34-45), for
// prefill and batched rows (M >= 8). Built as its own translation unit with
// -mllvm -amdgpu-mfma-vgpr-form=1, so that MFMA results land in ordinary
// vector registers, where the epilogue reads them.
//
// Arithmetic per output (m, n): t[b & 3] += (sa_b * sb_b) * (float)isum_b over
// the blocks b in order, no FMA, then y = ((t0 + t1) + t2) + t3. Every
// (row, column, block) therefore costs one rounded product of the two scales,
// one conversion, one rounded product and one rounded add; none of it can be
// folded into the integer accumulation, so the f32 epilogue, not the int8
// MFMA, bounds the kernel. Two matrix instructions take all they can of it:
//  * v_mfma_i32_32x32x32_i8 gives a 32 x 32 unit's exact block dots (isum),
//    one instruction per (unit, block);
//  * v_mfma_f32_32x32x1_2b_f32 gives two units' scale products sa * sb as
//    rank-1 outer products (a zero C and one nonzero product per output: the
//    correctly rounded f32 product, the rounding of the vector multiply).
// What remains on the vector unit is cvt, multiply and add: 3 operations per
// (row, column, block) instead of 4.
//
// Work split: the four partial sums t_j are independent chains (blocks
// b = j mod 4), so they are the unit of work. A workgroup owns a TM x TN
// output tile; each wave owns a 32 x 32 NJ sub-tile for CPW of the four
// chains. Both i8 operands of a 32x32x32 unit use the same byte map (lane l:
// row or column l % 32, bytes 16 (l / 32) .. +16 of the block), so the
// integer sum covers the block once. Accumulator v of lane l is output
// (row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32) of its unit; the f32
// outer product puts the scale product of the same output in the same
// register of its half.
//
// Operands are staged through LDS in chunks of KC blocks: every row's KC*32
// bytes by coalesced 16-byte loads, NS chunks ahead in registers, into a
// double-buffered tile whose rows are padded by 16 bytes (the fragment reads
// of 16 consecutive rows then cover all banks once), with the chunk's
// activation and weight scales beside it as f32. One barrier per chunk. The
// chains of an output meet at the end (in registers when one wave holds all
// four, else through LDS) and are summed as ((t0 + t1) + t2) + t3.
#include <hip/hip_runtime.h>

#include "kernrt_hip.h"
#include "device.hpp"
#include "kernels.hpp"
#include "numerics.hpp"

namespace kr {

typedef int g_v4i __attribute__((ext_vector_type(4)));
typedef int g_v16i __attribute__((ext_vector_type(16)));
typedef float g_v32f __attribute__((ext_vector_type(32)));

// Workgroup ids are dispatched round-robin over the 8 XCDs; consecutive
// logical tiles (the row tiles of one column tile) go to one XCD and share
// its L2.
__device__ __forceinline__ uint32_t gemm_xcd_tile(uint32_t id, uint32_t count) {
    const uint32_t per = count >> 3, rem = count & 7, xcd = id & 7, k = id >> 3;
    return xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
}

// SWI: the gate/up launch of a SwiGLU FFN with SiLU(gate) * up and its Q8
// blocks as the epilogue (silu_quant's arithmetic, elementwise.rs / quant.rs:
// 864-873): the tile's 64 columns are gate rows 32 t .. 32 t + 31 (ms.q[0])
// and up rows 32 t .. 32 t + 31 (ms.q[1]) of the same hidden block t, and the
// outputs are h's int8 quants and block scales in `so` instead of f32 gate/up,
// in chain-major block order when `cm` is set (for a chain-split down).
struct SwiOut {
    int8_t* q;
    float* s;
    uint16_t* h;
    uint32_t cm;
};

// ROPE: the q/k/v launch of a prefill with head_dim 64 (one head per 64-column
// tile) and the half-split RoPE layout: the epilogue rotates each q and k
// head's pairs (i, i + 32) at the row's position, as k_rope_kv does
// (cpu.rs:664-705), writes q to y[0], and k and v straight into the KV cache
// at the row's slot (kv_write, cpu.rs:563-573); y[1] and y[2] are not written.
struct RopeOut {
    const uint32_t* pos;    // [M] positions
    const uint32_t* slots;  // [M] cache slots
    const float2* tab;      // (cos, sin) per (position, pair): [pos][32]
    float* kc;              // the layer's keys: [seq_len][kv_dim]
    float* vc;              // and values
    uint32_t kv_dim;
};

// CS: the chain-split form for launches with few output tiles. Operands
// are chain-major (each row holds the blocks of chain 0 -- blocks 0, 4, 8,
// .. -- then those of chains 1, 2 and 3, with the scales in the same order),
// a workgroup runs one chain of one tile over that chain's contiguous quarter
// of K, all of its blocks into one accumulator in block order, and writes the
// chain's partial sums as plane `chain` of y ([4][M][ld]); the consumer adds
// the four planes as ((t0 + t1) + t2) + t3.
template <int SEM, int TM, int TN, int NJ, int CPW, int KC, int NS, int RS, int WPE, bool DBG, bool SWI = false,
          bool CS = false, bool ROPE = false>
__global__ __launch_bounds__(64 * (TM / 32) * (TN / (32 * NJ)) * (4 / CPW), WPE) void k_gemm_q8(
    MatSet ms, QuantAct x, uint32_t M, uint32_t K, uint32_t mtiles, int32_t* __restrict__ dbg, SwiOut so,
    RopeOut ro) {
    constexpr int WN = 32 * NJ, SM = TM / 32, NSUB = SM * (TN / WN), CG = 4 / CPW, NT = 64 * NSUB * CG;
    constexpr int ROW = KC * 32 + 16, PPR = KC * 2;
    constexpr int A_BYTES = TM * ROW, B_BYTES = TN * ROW;
    constexpr int BUF_BYTES = A_BYTES + B_BYTES + KC * (TM + TN) * 4;
    constexpr int PART_BYTES = CPW == 4 ? 0 : 4 * TM * TN * 4;
    constexpr int RING_BYTES = 3 * BUF_BYTES > PART_BYTES ? 3 * BUF_BYTES : PART_BYTES;
    constexpr int LDS_BYTES = RING_BYTES + (SWI ? 32 * 8 : 0);  // + the exp table
    constexpr int NQ = (TM + TN) * PPR, NP = (NQ + NT - 1) / NT;  // 16-byte pieces per chunk, per thread
    constexpr int NSC = ((TM + TN) * KC + NT - 1) / NT;         // scales per thread per chunk
    static_assert(TM % 32 == 0 && TN % WN == 0 && KC % (NJ == 2 || CPW >= 2 ? 4 : 8) == 0, "tile shape");
    static_assert(NJ == 1 || NJ == 2, "unit columns per wave");
    static_assert(CPW == 1 || CPW == 2 || CPW == 4, "chains per wave");
    static_assert(NT % PPR == 0, "a thread's pieces share their column");
    static_assert(!SWI || (TN == 64 && NJ == 2 && CPW < 4), "the SwiGLU epilogue needs one gate and one up unit per wave");
    static_assert(!CS || (CPW == 4 && !SWI && !DBG), "a chain-split wave runs its tile's one chain");
    static_assert(!ROPE || (TN == 64 && NJ == 2 && CPW < 4 && !SWI && !CS), "a RoPE tile is one 64-wide head");
    constexpr bool WF16 = SEM == SEM_FOUR_PARTIALS_F16;
    __shared__ __align__(16) int8_t lds[LDS_BYTES];
    uint64_t* const etab = (uint64_t*)(lds + RING_BYTES);
    auto sA = [&](int buf) { return lds + buf * BUF_BYTES; };
    auto sB = [&](int buf) { return lds + buf * BUF_BYTES + A_BYTES; };
    auto sX = [&](int buf) { return (float*)(lds + buf * BUF_BYTES + A_BYTES + B_BYTES); };  // [block][row]
    auto sW = [&](int buf) { return sX(buf) + KC * TM; };                                     // [block][col]

    // K: the row length (bytes, and 32 scales per block); nb: the blocks this
    // workgroup sums, from block koff / 32 of each row on (a chain's quarter
    // for CS)
    const uint32_t L = gemm_xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t mt = L % mtiles, chain = CS ? (L / mtiles) & 3 : 0, nt = CS ? L / mtiles / 4 : L / mtiles;
    const uint32_t nbr = K >> 5, nb = CS ? nbr / 4 : nbr, nchunks = (nb + KC - 1) / KC;
    const uint32_t kend = nb * 32, koff = chain * kend, soff = chain * nb;
    const int mi_ = SWI ? 0 : nt < ms.tile_end[0] ? 0 : (nt < ms.tile_end[1] ? 1 : 2);
    const uint32_t m0 = mt * TM, n0 = SWI ? nt * 32 : (nt - (mi_ == 0 ? 0 : ms.tile_end[mi_ > 0 ? mi_ - 1 : 0])) * TN;
    const int8_t* __restrict__ W = ms.q[mi_];
    const void* __restrict__ WS = ms.s[mi_];
    const uint32_t N = ms.n[mi_];
    const uint32_t tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, half = lane >> 5;
    if (SWI && tid < 32) etab[tid] = kExp2Tab[tid];  // read after the loop's barriers
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t cg = wave % CG, sub = wave / CG;                // chains cg*CPW .. +CPW-1
    const uint32_t wm0 = (sub % SM) * 32, wn0 = (sub / SM) * WN;  // the wave's sub-tile

    // loader map: piece q = tid + NT i is the 16-byte piece (row q / PPR,
    // column 16 (q % PPR)) of the A chunk for q < PPR TM, else of the B
    // chunk; scale s = tid + NT i is an activation scale (row s / KC, block
    // s % KC) for s < KC TM, else a weight scale. Rows past M or N read the
    // last row, blocks past the row end its last block.
    const int8_t* gp[NP];
    uint32_t lp[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const uint32_t q = min(tid + NT * i, (uint32_t)NQ - 1), isb = q >= PPR * TM;
        const uint32_t row = (isb ? q - PPR * TM : q) / PPR;
        if (SWI)  // B rows 0..31: gate, 32..63: up, of the hidden block's rows
            gp[i] = isb ? (row >= 32 ? ms.q[1] : ms.q[0]) + (size_t)min(n0 + (row & 31), N - 1) * K
                        : x.q + (size_t)min(m0 + row, M - 1) * K;
        else
            gp[i] = (isb ? W + (size_t)min(n0 + row, N - 1) * K : x.q + (size_t)min(m0 + row, M - 1) * K) + koff;
        lp[i] = (isb ? A_BYTES : 0) + row * ROW + (q % PPR) * 16;
    }
    const uint32_t pc = (tid % PPR) * 16;

    struct Stage {
        g_v4i p[NP];
        uint32_t sc[NSC];
    };
    auto gload = [&](Stage& st, uint32_t c) {
        c = c < nchunks ? c : nchunks - 1;
        const uint32_t col = min(c * KC * 32 + pc, kend - 16);  // past the end: a piece no block uses
#pragma unroll
        for (int i = 0; i < NP; i++) st.p[i] = *(const g_v4i*)(gp[i] + col);
#pragma unroll
        for (int i = 0; i < NSC; i++) {
            const uint32_t sidx = tid + NT * i;
            const uint32_t blk = soff + min(c * KC + sidx % KC, nb - 1);
            if (sidx < KC * TM) {
                st.sc[i] = f2u(x.s[(size_t)min(m0 + sidx / KC, M - 1) * nbr + blk]);
            } else if (sidx < KC * (TM + TN)) {
                const uint32_t col2 = (sidx - KC * TM) / KC;
                if (SWI)
                    st.sc[i] = scale_bits(WF16, col2 >= 32 ? ms.s[1] : ms.s[0],
                                          (size_t)min(n0 + (col2 & 31), N - 1) * nbr + blk);
                else
                    st.sc[i] = scale_bits(WF16, WS, (size_t)min(n0 + col2, N - 1) * nbr + blk);
            }
        }
    };
    auto lstore = [&](const Stage& st, int buf) {
#pragma unroll
        for (int i = 0; i < NP; i++)
            if (NQ % NT == 0 || i + 1 < NP || tid + NT * i < NQ) *(g_v4i*)(sA(buf) + lp[i]) = st.p[i];
#pragma unroll
        for (int i = 0; i < NSC; i++) {
            const uint32_t sidx = tid + NT * i, blk = sidx % KC;
            if (sidx < KC * TM)
                sX(buf)[blk * TM + sidx / KC] = u2f(st.sc[i]);
            else if (sidx < KC * (TM + TN))
                sW(buf)[blk * TN + (sidx - KC * TM) / KC] = scale_value(WF16, st.sc[i]);
        }
    };

    float t[CPW][NJ][16];
#pragma unroll
    for (int c2 = 0; c2 < CPW; c2++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) t[c2][j][v] = 0.0f;
    const g_v16i izero = {};
    const g_v32f fzero = {};

    // unit u of pair p (block within the chunk, chain slot, column half):
    // the two 32 x 32 units whose scale products one 2b instruction forms.
    //  * NJ == 2: both column halves of one block;
    //  * NJ == 1, CPW >= 2: one 128-byte group's blocks of two chains;
    //  * NJ == 1, CPW == 1: one chain's blocks in two consecutive groups.
    auto unit = [&](int p, int u, int& blk, int& c2, int& j) {
        if constexpr (NJ == 2) {
            const int h = p / CPW;
            c2 = p % CPW, j = u, blk = (int)cg * CPW + c2 + 4 * h;
        } else if constexpr (CPW >= 2) {
            const int h = p / (CPW / 2);
            c2 = 2 * (p % (CPW / 2)) + u, j = 0, blk = (int)cg * CPW + c2 + 4 * h;
        } else {
            c2 = 0, j = 0, blk = (int)cg + 4 * (2 * p + u);
        }
    };
    constexpr int PAIRS = NJ == 2 ? KC / 4 * CPW : KC * CPW / 8;
    static_assert(PAIRS > 0 && PAIRS % 2 == 0, "the register pipeline alternates two sets per pair");

    // One pair's operands (two i8 fragments per unit, the lane's 2b scale
    // operands) and results (the two units' block dots, their scale products).
    struct Ops {
        g_v4i a0, q0, a1, q1;
        float xs, ws;
    };
    struct Res {
        g_v32f P;
        g_v16i d0, d1;
    };
    auto ops_load = [&](Ops& o, int buf, int p) {
        int blk0, c20, j0, blk1, c21, j1;
        unit(p, 0, blk0, c20, j0);
        unit(p, 1, blk1, c21, j1);
        // the lane's half of the 2b operands: unit `half`'s activation scale
        // of row wm0 + r32 and weight scale of its column
        const int bh = half ? blk1 : blk0, jh = half ? j1 : j0;
        o.xs = sX(buf)[bh * TM + wm0 + r32];
        o.ws = sW(buf)[bh * TN + wn0 + 32 * jh + r32];
        o.a0 = *(const g_v4i*)(sA(buf) + (wm0 + r32) * ROW + blk0 * 32 + 16 * half);
        o.q0 = *(const g_v4i*)(sB(buf) + (wn0 + 32 * j0 + r32) * ROW + blk0 * 32 + 16 * half);
        if (blk1 != blk0) o.a1 = *(const g_v4i*)(sA(buf) + (wm0 + r32) * ROW + blk1 * 32 + 16 * half);
        o.q1 = *(const g_v4i*)(sB(buf) + (wn0 + 32 * j1 + r32) * ROW + blk1 * 32 + 16 * half);
    };
    auto mfma = [&](Res& r, const Ops& o, int p) {
        int blk0, c20, j0, blk1, c21, j1;
        unit(p, 0, blk0, c20, j0);
        unit(p, 1, blk1, c21, j1);
        r.P = __builtin_amdgcn_mfma_f32_32x32x1f32(o.xs, o.ws, fzero, 0, 0, 0);
        r.d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a0, o.q0, izero, 0, 0, 0);
        r.d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(blk1 != blk0 ? o.a1 : o.a0, o.q1, izero, 0, 0, 0);
    };
    auto epilogue = [&](const Res& r, uint32_t c, int p) {
        int blk0, c20, j0, blk1, c21, j1;
        unit(p, 0, blk0, c20, j0);
        unit(p, 1, blk1, c21, j1);
        const uint32_t b0 = c * KC + blk0, b1 = c * KC + blk1;
        if (b0 >= nb) return;  // blocks past the row end: staged copies, never summed
        if (DBG) {
            const uint32_t nn0 = n0 + wn0 + 32 * j0 + r32, nn1 = n0 + wn0 + 32 * j1 + r32;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t m = m0 + wm0 + 8 * (v >> 2) + 4 * half + (v & 3);
                if (m < M && nn0 < N) dbg[((size_t)m * N + nn0) * nb + b0] = r.d0[v];
                if (m < M && nn1 < N && b1 < nb) dbg[((size_t)m * N + nn1) * nb + b1] = r.d1[v];
            }
        }
        // dot.rs: t[b & 3] += (sa * sb) * (isum as f32); CS: every block is the chain's
#pragma unroll
        for (int v = 0; v < 16; v++) t[CS ? 0 : c20][j0][v] += r.P[v] * (float)r.d0[v];
        if (b1 < nb) {
#pragma unroll
            for (int v = 0; v < 16; v++) t[CS ? 0 : c21][j1][v] += r.P[16 + v] * (float)r.d1[v];
        }
    };

    // The chunk loop. LDS is a ring of three chunk buffers: at step c the
    // wave stores chunk c + 1 (its global loads issued NS steps earlier),
    // requests chunk c + 1 + NS, passes the barrier, and runs the pairs of
    // chunk c. A buffer is refilled two steps after its chunk was last read,
    // one barrier between, so the register pipeline below reads one chunk
    // ahead across the barrier: pair g's operands are read from LDS two
    // pairs ahead, its matrix instructions issued one pair ahead, and its
    // vector epilogue runs while the next pair's matrix work is in flight.
    // Chunks past the last one are staged copies of it (loads clamp), so the
    // look-ahead reads valid memory; their pairs are never summed.
    Stage st[NS];
#pragma unroll
    for (int s2 = 0; s2 < NS; s2++) gload(st[s2], s2);
    lstore(st[0], 0);
    gload(st[0], NS);
    __syncthreads();
    Ops o[2];
    Res rr[RS];
    ops_load(o[0], 0, 0);
    ops_load(o[1], 0, 1);
    if (RS == 2) mfma(rr[0], o[0], 0);
    uint32_t bc = 0, bn = 1, bf = 2;  // buffers of chunks c, c + 1, c + 2
    // One step: store chunk c + 1 (register stage (u + 1) % NS, a
    // compile-time index, so its load wait covers only that stage), request
    // chunk c + 1 + NS into the same stage, barrier, run chunk c's pairs.
    auto step = [&](uint32_t c, int u) {
        lstore(st[(u + 1) % NS], bn);
        gload(st[(u + 1) % NS], c + 1 + NS);
        __syncthreads();
#pragma unroll
        for (int p = 0; p < PAIRS; p++) {
            if constexpr (RS == 1) {
                // pair p's matrix work, pair p + 2's operands into the set it
                // read, then pair p's epilogue
                mfma(rr[0], o[p & 1], p);
                if (p + 2 < PAIRS)
                    ops_load(o[p & 1], bc, p + 2);
                else
                    ops_load(o[p & 1], bn, p + 2 - PAIRS);
                epilogue(rr[0], c, p);
            } else {
                // pair p + 2 (maybe in chunk c + 1) into the operand set pair p used
                if (p + 2 < PAIRS)
                    ops_load(o[p & 1], bc, p + 2);
                else
                    ops_load(o[p & 1], bn, p + 2 - PAIRS);
                // pair p + 1's matrix work, then pair p's epilogue
                mfma(rr[(p + 1) & 1], o[(p + 1) & 1], (p + 1) % PAIRS);
                epilogue(rr[p & 1], c, p);
            }
        }
        const uint32_t t0 = bc;
        bc = bn, bn = bf, bf = t0;
    };
    // full groups of NS steps, then the remaining nchunks % NS steps (each
    // still with its compile-time stage)
    const uint32_t full = nchunks / NS * NS;
    uint32_t c0 = 0;
    for (; c0 < full; c0 += NS) {
#pragma unroll
        for (int u = 0; u < NS; u++) step(c0 + u, u);
    }
#pragma unroll
    for (int u = 0; u < NS; u++)
        if (c0 + u < nchunks) step(c0 + u, u);
    __syncthreads();  // the partial-sum exchange below reuses the ring

    float* Y = ms.y[mi_];
    const uint32_t ld = ms.ld[mi_];
    if constexpr (CS) {
        // the chain's partial sums, plane `chain`
        float* P = Y + (size_t)chain * M * ld;
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t m = m0 + wm0 + 8 * (v >> 2) + 4 * half + (v & 3), n = n0 + wn0 + 32 * j + r32;
                if (m < M && n < N) P[(size_t)m * ld + n] = t[0][j][v];
            }
    } else if constexpr (CPW == 4) {
        // one wave holds all four chains of its outputs
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t m = m0 + wm0 + 8 * (v >> 2) + 4 * half + (v & 3), n = n0 + wn0 + 32 * j + r32;
                if (m < M && n < N) Y[(size_t)m * ld + n] = ((t[0][j][v] + t[1][j][v]) + t[2][j][v]) + t[3][j][v];
            }
    } else {
        // the chains meet in LDS, four consecutive accumulators per lane as
        // one 16-byte store: part[chain][sub][j][v / 4][lane][v % 4]
        constexpr int WOUT = 32 * WN;
        float4* part = (float4*)lds;
#pragma unroll
        for (int c2 = 0; c2 < CPW; c2++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int v4 = 0; v4 < 4; v4++)
                    part[(((cg * CPW + c2) * NSUB + sub) * WOUT) / 4 + (j * 4 + v4) * 64 + lane] =
                        float4{t[c2][j][4 * v4], t[c2][j][4 * v4 + 1], t[c2][j][4 * v4 + 2], t[c2][j][4 * v4 + 3]};
        __syncthreads();
        auto sum4 = [&](uint32_t o4) {
            const float4 p0 = part[o4], p1 = part[TM * TN / 4 + o4], p2 = part[2 * TM * TN / 4 + o4];
            const float4 p3 = part[3 * TM * TN / 4 + o4];
            return float4{((p0.x + p1.x) + p2.x) + p3.x, ((p0.y + p1.y) + p2.y) + p3.y,
                          ((p0.z + p1.z) + p2.z) + p3.z, ((p0.w + p1.w) + p2.w) + p3.w};
        };
        if constexpr (SWI) {
            // element e: (sub, v4, lane): rows 8 v4 + 4 (lane / 32) + 0..3 of
            // hidden column n0 + lane % 32, its gate (unit 0) and up (unit 1);
            // the 32 lanes of a half-wave hold one row's Q8 block
            const uint32_t nbh = N >> 5, pb = so.cm ? cm_block(n0 >> 5, nbh) : n0 >> 5;
#pragma unroll
            for (int k = 0; k < TM * 8 / NT; k++) {
                const uint32_t e = tid + NT * k, sb = e >> 8, v4 = (e >> 6) & 3, l = e & 63;
                const uint32_t og = sb * (WOUT / 4) + v4 * 64 + l;
                const float4 g4 = sum4(og), u4 = sum4(og + 256);
                const float gv[4] = {g4.x, g4.y, g4.z, g4.w}, uv[4] = {u4.x, u4.y, u4.z, u4.w};
                const uint32_t mb = m0 + (sb % SM) * 32 + 8 * v4 + 4 * (l >> 5), col = n0 + (l & 31);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const bool live = mb + r < M;
                    // cpu.rs:708-710: silu(g) * u
                    const float h = div_rn(gv[r], 1.0f + glibc_expf(-gv[r], etab)) * uv[r];
                    const size_t orow = live ? mb + r : 0, oi = orow * N + pb * 32 + (col & 31);
                    quant_lane(h, live, so.q + oi, so.s + orow * nbh + pb, so.h + orow * nbh + pb);
                }
            }
            return;
        }
        if constexpr (ROPE) {
            // element e: (sub, v4, lane): rows 8 v4 + 4 (lane / 32) + 0..3 of
            // the head's columns i = lane % 32 (unit 0) and i + 32 (unit 1)
#pragma unroll
            for (int k = 0; k < TM * 8 / NT; k++) {
                const uint32_t e = tid + NT * k, sb = e >> 8, v4 = (e >> 6) & 3, l = e & 63;
                const uint32_t og = sb * (WOUT / 4) + v4 * 64 + l;
                const float4 a4 = sum4(og), b4 = sum4(og + 256);
                const float av[4] = {a4.x, a4.y, a4.z, a4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
                const uint32_t mb = m0 + (sb % SM) * 32 + 8 * v4 + 4 * (l >> 5), i = l & 31, c0 = n0 + i;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if (mb + r >= M) continue;
                    const uint32_t m = mb + r;
                    if (mi_ == 2) {  // v: to the cache as it is
                        float* vr = ro.vc + (size_t)ro.slots[m] * ro.kv_dim;
                        vr[c0] = av[r];
                        vr[c0 + 32] = bv[r];
                        continue;
                    }
                    // k_rope_kv: r0 = a cos - b sin, r1 = a sin + b cos
                    const float2 cs = ro.tab[(size_t)ro.pos[m] * 32 + i];
                    const float r0 = av[r] * cs.x - bv[r] * cs.y;
                    const float r1 = av[r] * cs.y + bv[r] * cs.x;
                    float* dst = mi_ == 0 ? Y + (size_t)m * ld : ro.kc + (size_t)ro.slots[m] * ro.kv_dim;
                    dst[c0] = r0;
                    dst[c0 + 32] = r1;
                }
            }
            return;
        }
        // element o4 of a plane: (sub, j, v4, lane), the 4 outputs rows
        // 8 v4 + 4 (lane / 32) + 0..3 of column lane % 32
#pragma unroll
        for (int k = 0; k < TM * TN / 4 / NT; k++) {
            const uint32_t o4 = tid + NT * k, sb = o4 / (WOUT / 4), oo = o4 % (WOUT / 4);
            const uint32_t l = oo & 63, jv = oo >> 6, j = jv >> 2, v4 = jv & 3;
            const uint32_t mb = m0 + (sb % SM) * 32 + 8 * v4 + 4 * (l >> 5);
            const uint32_t n = n0 + (sb / SM) * WN + 32 * j + (l & 31);
            const float4 p0 = part[o4], p1 = part[TM * TN / 4 + o4], p2 = part[2 * TM * TN / 4 + o4];
            const float4 p3 = part[3 * TM * TN / 4 + o4];
            if (n < N) {
                if (mb < M) Y[(size_t)mb * ld + n] = ((p0.x + p1.x) + p2.x) + p3.x;
                if (mb + 1 < M) Y[(size_t)(mb + 1) * ld + n] = ((p0.y + p1.y) + p2.y) + p3.y;
                if (mb + 2 < M) Y[(size_t)(mb + 2) * ld + n] = ((p0.z + p1.z) + p2.z) + p3.z;
                if (mb + 3 < M) Y[(size_t)(mb + 3) * ld + n] = ((p0.w + p1.w) + p2.w) + p3.w;
            }
        }
    }
}

template <int SEM, int TM, int TN, int NJ, int CPW, int KC, int NS, int RS, int WPE>
static void launch_q8(hipStream_t st, MatSet ms, QuantAct x, size_t rows, size_t k, int32_t* dbg) {
    uint32_t total = 0;
    for (int i = 0; i < 3; i++) {
        if (i < ms.count) total += (uint32_t)((ms.n[i] + TN - 1) / TN);
        ms.tile_end[i] = total;
    }
    const uint32_t mtiles = (uint32_t)((rows + TM - 1) / TM);
    const dim3 grid(total * mtiles), block(64 * (TM / 32) * (TN / (32 * NJ)) * (4 / CPW));
    if (dbg)
        hipLaunchKernelGGL((k_gemm_q8<SEM, TM, TN, NJ, CPW, KC, NS, RS, WPE, true>), grid, block, 0, st, ms, x,
                           (uint32_t)rows, (uint32_t)k, mtiles, dbg, SwiOut{}, RopeOut{});
    else
        hipLaunchKernelGGL((k_gemm_q8<SEM, TM, TN, NJ, CPW, KC, NS, RS, WPE, false>), grid, block, 0, st, ms, x,
                           (uint32_t)rows, (uint32_t)k, mtiles, dbg, SwiOut{}, RopeOut{});
}

// The chain-split form: tiles x 4 chains; y[0] receives [4][rows][ld].
template <int TM, int TN, int NJ, int KC, int NS, int RS, int WPE>
static void launch_q8_cs(hipStream_t st, MatSet ms, QuantAct x, size_t rows, size_t k) {
    const uint32_t ntiles = (ms.n[0] + TN - 1) / TN, mtiles = (uint32_t)((rows + TM - 1) / TM);
    ms.tile_end[0] = ms.tile_end[1] = ms.tile_end[2] = ntiles;
    const dim3 grid(ntiles * 4 * mtiles), block(64 * (TM / 32) * (TN / (32 * NJ)));
    hipLaunchKernelGGL((k_gemm_q8<SEM_FOUR_PARTIALS_F32, TM, TN, NJ, 4, KC, NS, RS, WPE, false, false, true>), grid,
                       block, 0, st, ms, x, (uint32_t)rows, (uint32_t)k, mtiles, nullptr, SwiOut{}, RopeOut{});
}

// The SwiGLU form: one tile per (row block, hidden block of 32).
template <int TM, int NJ, int CPW, int KC, int NS, int RS, int WPE>
static void launch_q8_swi(hipStream_t st, const MatSet& ms, QuantAct x, size_t rows, size_t k, SwiOut so) {
    const uint32_t mtiles = (uint32_t)((rows + TM - 1) / TM), ntiles = ms.n[0] / 32;
    const dim3 grid(ntiles * mtiles), block(64 * (TM / 32) * (64 / (32 * NJ)) * (4 / CPW));
    hipLaunchKernelGGL((k_gemm_q8<SEM_FOUR_PARTIALS_F32, TM, 64, NJ, CPW, KC, NS, RS, WPE, false, true>), grid, block,
                       0, st, ms, x, (uint32_t)rows, (uint32_t)k, mtiles, nullptr, so, RopeOut{});
}

// The narrow form (few column tiles: o and down at N = 2048), on 16x16x32
// int8 MFMA with the whole epilogue on the vector unit. The
// reference's four partial sums t[j] (blocks b with b % 4 == j, in order) are
// independent chains, so they are the unit of work: a workgroup owns a TM x TN
// output tile, and each of its waves runs CPW of the four chains over a
// WM x WN sub-tile. Per block a wave reads one A fragment and four activation
// scales per 16-row slice and one B fragment and one weight scale per
// 16-column slice from LDS and reuses them across the other dimension, so the
// LDS read traffic per output falls with the sub-tile size and the per-block
// f32 epilogue (cvt, two multiplies, add: 4 VALU operations per output)
// dominates the instruction stream. Chunks of KC blocks of the A and B rows
// and their scales are staged through a double-buffered, padded LDS tile, NS
// chunks ahead in registers. At the end the chains of every output meet --
// in registers when one wave holds all four, else in LDS -- and are summed as
// ((t0 + t1) + t2) + t3.
template <int SEM, int TM, int TN, int WM, int WN, int CPW, int KC, int NS, int WPE, bool DBG>
__global__ __launch_bounds__(64 * (TM / WM) * (TN / WN) * (4 / CPW), WPE) void k_gemm_q8_s16(MatSet ms, QuantAct x,
                                                                                 uint32_t M, uint32_t K,
                                                                                 uint32_t mtiles,
                                                                                 int32_t* __restrict__ dbg) {
    constexpr int ROW = KC * 32 + 16, PPR = KC * 2, MI = WM / 16, NI = WN / 16, CG = 4 / CPW;
    constexpr int SM = TM / WM, NSUB = SM * (TN / WN), NT = 64 * NSUB * CG;
    constexpr int A_BYTES = TM * ROW, B_BYTES = TN * ROW;
    constexpr int BUF_BYTES = A_BYTES + B_BYTES + KC * (TM + TN) * 4;
    constexpr int PART_BYTES = CPW == 4 ? 0 : 4 * TM * TN * 4;
    constexpr int LDS_BYTES = 2 * BUF_BYTES > PART_BYTES ? 2 * BUF_BYTES : PART_BYTES;
    constexpr int NQ = (TM + TN) * PPR, NP = (NQ + NT - 1) / NT;  // 16-byte pieces per chunk, per thread
    constexpr int NSC = ((TM + TN) * KC + NT - 1) / NT;  // scales per thread per chunk
    static_assert(WM % 16 == 0 && WN % 16 == 0 && TM % WM == 0 && TN % WN == 0 && KC % 4 == 0, "tile shape");
    static_assert(CPW == 1 || CPW == 2 || CPW == 4, "chains per wave");
    static_assert(NT % PPR == 0, "a thread's pieces share their column");
    __shared__ __align__(16) int8_t lds[LDS_BYTES];
    auto sA = [&](int buf) { return lds + buf * BUF_BYTES; };
    auto sB = [&](int buf) { return lds + buf * BUF_BYTES + A_BYTES; };
    auto sX = [&](int buf) { return (float*)(lds + buf * BUF_BYTES + A_BYTES + B_BYTES); };  // [block][row]
    auto sW = [&](int buf) { return sX(buf) + KC * TM; };                                     // [block][col]

    const uint32_t nb = K >> 5, nchunks = (nb + KC - 1) / KC;
    const uint32_t L = gemm_xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t mt = L % mtiles, nt = L / mtiles;
    const int mi_ = nt < ms.tile_end[0] ? 0 : (nt < ms.tile_end[1] ? 1 : 2);
    const uint32_t m0 = mt * TM, n0 = (nt - (mi_ == 0 ? 0 : ms.tile_end[mi_ - 1])) * TN;
    const int8_t* __restrict__ W = ms.q[mi_];
    const void* __restrict__ WS = ms.s[mi_];
    const uint32_t N = ms.n[mi_];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t cg = wave % CG, sub = wave / CG;                // chains cg*CPW .. +CPW-1
    const uint32_t wm0 = (sub % SM) * WM, wn0 = (sub / SM) * WN;  // the wave's sub-tile
    const uint32_t r = lane & 15, quad = lane >> 4;
    constexpr bool WF16 = SEM == SEM_FOUR_PARTIALS_F16;

    // loader map: piece q = tid + NT i is the 16-byte piece (row q / PPR,
    // column 16 (q % PPR)) of the A chunk for q < PPR TM, else of the B
    // chunk; scale s = tid + NT i is an activation scale (row s / KC, block
    // s % KC) for s < KC TM, else a weight scale. Rows past M or N read the
    // last row, blocks past the row end its last block.
    const int8_t* gp[NP];
    uint32_t lp[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const uint32_t q = min(tid + NT * i, (uint32_t)NQ - 1), isb = q >= PPR * TM;
        const uint32_t row = (isb ? q - PPR * TM : q) / PPR;
        gp[i] = isb ? W + (size_t)min(n0 + row, N - 1) * K : x.q + (size_t)min(m0 + row, M - 1) * K;
        lp[i] = (isb ? A_BYTES : 0) + row * ROW + (q % PPR) * 16;
    }
    const uint32_t pc = (tid % PPR) * 16;

    struct Stage {
        g_v4i p[NP];
        uint32_t sc[NSC];
    };
    auto gload = [&](Stage& st, uint32_t c) {
        c = c < nchunks ? c : nchunks - 1;
        const uint32_t col = min(c * KC * 32 + pc, K - 16);  // past the row end: a piece no block uses
#pragma unroll
        for (int i = 0; i < NP; i++) st.p[i] = *(const g_v4i*)(gp[i] + col);
#pragma unroll
        for (int i = 0; i < NSC; i++) {
            const uint32_t sidx = tid + NT * i;
            const uint32_t blk = min(c * KC + sidx % KC, nb - 1);
            if (sidx < KC * TM) {
                st.sc[i] = f2u(x.s[(size_t)min(m0 + sidx / KC, M - 1) * nb + blk]);
            } else if (sidx < KC * (TM + TN)) {
                const uint32_t col2 = (sidx - KC * TM) / KC;
                st.sc[i] = scale_bits(WF16, WS, (size_t)min(n0 + col2, N - 1) * nb + blk);
            }
        }
    };
    auto lstore = [&](const Stage& st, int buf) {
#pragma unroll
        for (int i = 0; i < NP; i++)
            if (NQ % NT == 0 || i + 1 < NP || tid + NT * i < NQ) *(g_v4i*)(sA(buf) + lp[i]) = st.p[i];
#pragma unroll
        for (int i = 0; i < NSC; i++) {
            const uint32_t sidx = tid + NT * i, blk = sidx % KC;
            if (sidx < KC * TM)
                sX(buf)[blk * TM + sidx / KC] = u2f(st.sc[i]);
            else if (sidx < KC * (TM + TN))
                sW(buf)[blk * TN + (sidx - KC * TM) / KC] = scale_value(WF16, st.sc[i]);
        }
    };

    float t[CPW][MI][NI][4];
#pragma unroll
    for (int c2 = 0; c2 < CPW; c2++)
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < NI; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) t[c2][i][j][v] = 0.0f;
    const g_v4i zero = {0, 0, 0, 0};
    auto compute = [&](int buf, uint32_t c) {
#pragma unroll
        for (int h = 0; h < KC / 4; h++)
#pragma unroll
            for (int c2 = 0; c2 < CPW; c2++) {
                const uint32_t blk = cg * CPW + c2 + 4 * h, b = c * KC + blk;
                if (b >= nb) break;
                long a[MI], bq[NI];
                float w[NI];
                float4 xs[MI];
#pragma unroll
                for (int i = 0; i < MI; i++) {
                    a[i] = *(const long*)(sA(buf) + (wm0 + i * 16 + r) * ROW + blk * 32 + 8 * quad);
                    xs[i] = *(const float4*)(sX(buf) + blk * TM + wm0 + i * 16 + 4 * quad);
                }
#pragma unroll
                for (int j = 0; j < NI; j++) {
                    bq[j] = *(const long*)(sB(buf) + (wn0 + j * 16 + r) * ROW + blk * 32 + 8 * quad);
                    w[j] = sW(buf)[blk * TN + wn0 + j * 16 + r];
                }
#pragma unroll
                for (int i = 0; i < MI; i++)
#pragma unroll
                    for (int j = 0; j < NI; j++) {
                        const g_v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], bq[j], zero, 0, 0, 0);
                        if (DBG) {
                            const uint32_t n = n0 + wn0 + j * 16 + r;
#pragma unroll
                            for (int v = 0; v < 4; v++) {
                                const uint32_t m = m0 + wm0 + i * 16 + 4 * quad + v;
                                if (m < M && n < N) dbg[((size_t)m * N + n) * nb + b] = d[v];
                            }
                        }
                        // dot.rs: t[b & 3] += (sa * sb) * (isum as f32)
                        t[c2][i][j][0] += (w[j] * xs[i].x) * (float)d[0];
                        t[c2][i][j][1] += (w[j] * xs[i].y) * (float)d[1];
                        t[c2][i][j][2] += (w[j] * xs[i].z) * (float)d[2];
                        t[c2][i][j][3] += (w[j] * xs[i].w) * (float)d[3];
                    }
            }
    };

    gemm_pipeline<NS, Stage>(nchunks, gload, lstore, compute);

    float* Y = ms.y[mi_];
    const uint32_t ld = ms.ld[mi_];
    if constexpr (CPW == 4) {
        // one wave holds all four chains of its outputs
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < NI; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const uint32_t m = m0 + wm0 + i * 16 + 4 * quad + v, n = n0 + wn0 + j * 16 + r;
                    if (m < M && n < N)
                        Y[(size_t)m * ld + n] = ((t[0][i][j][v] + t[1][i][j][v]) + t[2][i][j][v]) + t[3][i][j][v];
                }
    } else {
        // the chains meet in LDS: part[chain][sub][((i * NI + j) * 4 + v) * 64 + lane]
        constexpr int WOUT = WM * WN;
        float* part = (float*)lds;
#pragma unroll
        for (int c2 = 0; c2 < CPW; c2++)
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NI; j++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        part[((cg * CPW + c2) * NSUB + sub) * WOUT + ((i * NI + j) * 4 + v) * 64 + lane] =
                            t[c2][i][j][v];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < TM * TN / NT; k++) {
            const uint32_t o = tid + NT * k, sb = o / WOUT, oo = o % WOUT;
            const uint32_t l = oo & 63, v = (oo >> 6) & 3, ij = oo >> 8, i = ij / NI, j = ij % NI;
            const uint32_t m = m0 + (sb % SM) * WM + i * 16 + 4 * (l >> 4) + v;
            const uint32_t n = n0 + (sb / SM) * WN + j * 16 + (l & 15);
            if (m < M && n < N) {
                const float p0 = part[o], p1 = part[TM * TN + o], p2 = part[2 * TM * TN + o];
                const float p3 = part[3 * TM * TN + o];
                Y[(size_t)m * ld + n] = ((p0 + p1) + p2) + p3;
            }
        }
    }
}

template <int SEM, int TM, int TN, int WM, int WN, int CPW, int KC, int NS, int WPE>
static void launch_q8_s16(hipStream_t st, MatSet ms, QuantAct x, size_t rows, size_t k, int32_t* dbg) {
    uint32_t total = 0;
    for (int i = 0; i < 3; i++) {
        if (i < ms.count) total += (uint32_t)((ms.n[i] + TN - 1) / TN);
        ms.tile_end[i] = total;
    }
    const uint32_t mtiles = (uint32_t)((rows + TM - 1) / TM);
    const dim3 grid(total * mtiles), block(64 * (TM / WM) * (TN / WN) * (4 / CPW));
    if (dbg)
        hipLaunchKernelGGL((k_gemm_q8_s16<SEM, TM, TN, WM, WN, CPW, KC, NS, WPE, true>), grid, block, 0, st, ms, x,
                           (uint32_t)rows, (uint32_t)k, mtiles, dbg);
    else
        hipLaunchKernelGGL((k_gemm_q8_s16<SEM, TM, TN, WM, WN, CPW, KC, NS, WPE, false>), grid, block, 0, st, ms, x,
                           (uint32_t)rows, (uint32_t)k, mtiles, dbg);
}

// Column tiles of width tn over the set's matrices.
static uint32_t gemm_col_tiles(const MatSet& ms, uint32_t tn) {
    uint32_t n = 0;
    for (int i = 0; i < ms.count; i++) n += (ms.n[i] + tn - 1) / tn;
    return n;
}

template <int SEM>
static hipError_t gemm_q8_go(hipStream_t st, const MatSet& ms, size_t k, QuantAct x, size_t rows, int32_t* dbg) {
    // the widest tile that still gives the grid enough workgroups: wider
    // tiles stage fewer bytes per output (A and B rows are shared by more
    // outputs) but give fewer, longer workgroups
    const size_t m128 = (rows + 127) / 128, m64 = (rows + 63) / 64;
    if (rows > 64 && m128 * gemm_col_tiles(ms, 64) >= 200)
        launch_q8<SEM, 128, 64, 2, 2, 4, 3, 1, 1>(st, ms, x, rows, k, dbg);
    else if (m64 * gemm_col_tiles(ms, 64) >= 160)
        launch_q8<SEM, 64, 64, 2, 1, 8, 2, 2, 1>(st, ms, x, rows, k, dbg);
    else
        launch_q8_s16<SEM, 32, 32, 16, 16, 1, 8, 4, 1>(st, ms, x, rows, k, dbg);
    return hipGetLastError();
}

// Whether the q/k/v GEMM with the RoPE and kv_write epilogue applies: Q8_0,
// head_dim 64 whole heads, and a row count at which the plain launch takes
// the 64x64 tiles (the form the epilogue is built in).
bool qkv_rope_q8_ok(const DevMatrix& q, const DevMatrix& k, const DevMatrix& v, size_t rows) {
    if (q.storage != KR_STORAGE_Q8_0 || k.storage != KR_STORAGE_Q8_0 || v.storage != KR_STORAGE_Q8_0) return false;
    if (q.k != k.k || q.k != v.k || k.n != v.n || q.n % 64 != 0 || k.n % 64 != 0 || rows < 8) return false;
    const size_t tiles = (q.n + k.n + v.n) / 64, m128 = (rows + 127) / 128, m64 = (rows + 63) / 64;
    return !(rows > 64 && m128 * tiles >= 200) && m64 * tiles >= 160;
}

hipError_t launch_qkv_rope_q8(hipStream_t st, const DevMatrix& q, const DevMatrix& k, const DevMatrix& v, QuantAct x,
                              size_t rows, float* yq, const uint32_t* pos, const uint32_t* slots, const float2* tab,
                              float* kc, float* vc) {
    if (!qkv_rope_q8_ok(q, k, v, rows)) return hipErrorInvalidValue;
    MatSet ms{};
    const DevMatrix* w[3] = {&q, &k, &v};
    uint32_t total = 0;
    for (int i = 0; i < 3; i++) {
        ms.q[i] = w[i]->q, ms.s[i] = w[i]->s, ms.n[i] = (uint32_t)w[i]->n;
        total += (uint32_t)(w[i]->n / 64);
        ms.tile_end[i] = total;
    }
    ms.y[0] = yq, ms.ld[0] = (uint32_t)q.n;
    ms.count = 3;
    const RopeOut ro{pos, slots, tab, kc, vc, (uint32_t)k.n};
    const uint32_t mtiles = (uint32_t)((rows + 63) / 64);
    hipLaunchKernelGGL((k_gemm_q8<SEM_FOUR_PARTIALS_F32, 64, 64, 2, 1, 8, 2, 2, 1, false, false, false, true>),
                       dim3(total * mtiles), dim3(64 * 2 * 1 * 4), 0, st, ms, x, (uint32_t)rows, (uint32_t)q.k, mtiles,
                       nullptr, SwiOut{}, ro);
    return hipGetLastError();
}

// One v_mfma_f32_32x32x1_2b_f32 per wave on given operands: lane l brings
// a[g][l] and b[g][l] (block l / 32, row or column l % 32) and its 32
// accumulator registers c[g][v][l]; out[g][v][l] is register v afterwards.
// The GEMM's scale products and the prefill attention's chains rely on each
// output being fmaf(a, b, c) of its operands; this lets a test check that.
__global__ __launch_bounds__(64) void k_mfma_f32_probe(const float* __restrict__ a, const float* __restrict__ b,
                                                       const float* __restrict__ c, float* __restrict__ out) {
    const uint32_t g = blockIdx.x, l = threadIdx.x;
    g_v32f acc;
#pragma unroll
    for (int v = 0; v < 32; v++) acc[v] = c[((size_t)g * 32 + v) * 64 + l];
    acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a[(size_t)g * 64 + l], b[(size_t)g * 64 + l], acc, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 32; v++) out[((size_t)g * 32 + v) * 64 + l] = acc[v];
}

hipError_t launch_mfma_f32_probe(hipStream_t st, const float* a, const float* b, const float* c, float* out,
                                 size_t groups) {
    hipLaunchKernelGGL(k_mfma_f32_probe, dim3((unsigned)groups), dim3(64), 0, st, a, b, c, out);
    return hipGetLastError();
}

hipError_t launch_gate_up_silu_q8(hipStream_t st, const DevMatrix& gate, const DevMatrix& up, QuantAct x, size_t rows,
                                  int8_t* hq, float* hs, uint16_t* hh, bool chain_major) {
    if (gate.storage != KR_STORAGE_Q8_0 || up.storage != KR_STORAGE_Q8_0 || gate.n != up.n || gate.k != up.k ||
        gate.n % 32 != 0 || rows == 0 || (chain_major && gate.n % 128 != 0))
        return hipErrorInvalidValue;
    MatSet ms{};
    ms.q[0] = gate.q, ms.q[1] = up.q;
    ms.s[0] = gate.s, ms.s[1] = up.s;
    ms.n[0] = ms.n[1] = (uint32_t)gate.n;
    ms.count = 2;
    const SwiOut so{hq, hs, hh, chain_major ? 1u : 0u};
    const size_t m128 = (rows + 127) / 128, blocks = gate.n / 32;
    if (rows > 64 && m128 * blocks >= 200)
        launch_q8_swi<128, 2, 2, 4, 3, 1, 1>(st, ms, x, rows, gate.k, so);
    else
        launch_q8_swi<64, 2, 1, 8, 2, 2, 1>(st, ms, x, rows, gate.k, so);
    return hipGetLastError();
}

// The chain-major copy of a Q8_0 matrix: each row's blocks reordered by
// cm_block, scales with them. One thread per 16-byte half block.
__global__ __launch_bounds__(256) void k_chain_major(const int8_t* __restrict__ q, const float* __restrict__ s,
                                                     int8_t* __restrict__ cq, float* __restrict__ cs, uint32_t nb,
                                                     size_t pieces) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pieces) return;
    const size_t row = i / (2 * nb);
    const uint32_t rem = (uint32_t)(i - row * 2 * nb), b = rem >> 1, h = rem & 1, p = cm_block(b, nb);
    const size_t rb = row * nb;
    *(g_v4i*)(cq + (rb + p) * 32 + 16 * h) = *(const g_v4i*)(q + (rb + b) * 32 + 16 * h);
    if (h == 0) cs[rb + p] = s[rb + b];
}

hipError_t launch_chain_major(hipStream_t st, const DevMatrix& m, int8_t* cq, float* cs) {
    if (m.storage != KR_STORAGE_Q8_0 || m.k % 128 != 0) return hipErrorInvalidValue;
    const uint32_t nb = (uint32_t)(m.k / 32);
    const size_t pieces = m.n * nb * 2;
    hipLaunchKernelGGL(k_chain_major, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, st, m.q,
                       (const float*)m.s, cq, cs, nb, pieces);
    return hipGetLastError();
}

hipError_t launch_gemm_q8_cs(hipStream_t st, const DevMatrix& cm, QuantAct x, size_t rows, float* y4) {
    if (cm.storage != KR_STORAGE_Q8_0 || cm.k % 128 != 0 || rows == 0) return hipErrorInvalidValue;
    MatSet ms{};
    ms.q[0] = cm.q, ms.s[0] = cm.s, ms.y[0] = y4, ms.n[0] = (uint32_t)cm.n, ms.ld[0] = (uint32_t)cm.n;
    ms.count = 1;
    launch_q8_cs<64, 64, 1, 4, 3, 2, 1>(st, ms, x, rows, cm.k);
    return hipGetLastError();
}

hipError_t launch_gemm_q8(hipStream_t st, int sem, const MatSet& ms, size_t k, QuantAct x, size_t rows,
                          int32_t* dbg) {
    if (sem == SEM_FOUR_PARTIALS_F32) return gemm_q8_go<SEM_FOUR_PARTIALS_F32>(st, ms, k, x, rows, dbg);
    if (sem == SEM_FOUR_PARTIALS_F16) return gemm_q8_go<SEM_FOUR_PARTIALS_F16>(st, ms, k, x, rows, dbg);
    return hipErrorInvalidValue;
}

}  // namespace kr

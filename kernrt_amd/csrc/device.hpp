// Device helpers shared by the kernel sources of the HIP backend.
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "numerics.hpp"

namespace kr {

// Correctly rounded f32 division and square root, as the reference's x86 SSE
// arithmetic gives. The IEEE double operation rounded once to f32 is the
// correctly rounded f32 result (53 >= 2*24 + 2 makes the double rounding
// innocuous for / and sqrt); the f32 library forms are not exact here.
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }
__device__ __forceinline__ float sqrt_rn(float a) { return (float)__builtin_sqrt((double)a); }

// NaN-ignoring max across lanes with DPP (a few cycles per step, no LDS
// round trip as with __shfl_xor). Max is order-free, so every grouping gives
// the same result.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_max_step(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xf,
                                                               false)));
}
// max over each aligned group of 8 / 16 / 32 lanes, in every lane of the group
__device__ __forceinline__ float group_max8(float v) {
    v = dpp_max_step<0xB1, 0xf>(v);      // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xf>(v);      // quad_perm [2,3,0,1]
    return dpp_max_step<0x141, 0xf>(v);  // row_half_mirror
}
__device__ __forceinline__ float group_max16(float v) { return dpp_max_step<0x140, 0xf>(group_max8(v)); }  // row_mirror
__device__ __forceinline__ float group_max32(float v) {
    v = group_max16(v);  // then lane ^ 16 within the 32-lane group (ds_swizzle bit mode)
    return fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
}

// NaN-ignoring max over the 64 lanes of a wave, returned to every lane: DPP
// swaps within quads, half-rows and rows, then row broadcasts 15 and 31 into
// lane 63 (a few cycles each, no LDS round trip). Max is order-free.
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max_step<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_max_step<0x141, 0xf>(v);  // row_half_mirror
    v = dpp_max_step<0x140, 0xf>(v);  // row_mirror
    v = dpp_max_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    v = dpp_max_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// f32 -> IEEE binary16 bits, round to nearest even, as f32_to_f16_bits
// (quant.rs:722-758): the hardware conversion gives the same bits for every
// non-NaN input (all 2^32 inputs compared on gfx950); NaN keeps the software
// routine's quiet-NaN pattern. A couple of instructions instead of a branchy
// integer routine on the quantizers' critical path.
__device__ __forceinline__ uint16_t f16_bits(float v) {
    const uint32_t b = f2u(v);
    const uint16_t hw = __builtin_bit_cast(uint16_t, (_Float16)v);
    return (b & 0x7fffffffu) > 0x7f800000u ? (uint16_t)(((b >> 16) & 0x8000u) | 0x7e00u) : hw;
}

// Quantize one f32 value per lane as part of a 32-lane Q8 block (lanes
// 32k..32k+31 hold one block), exactly as Q8Vec::quantize_into does
// (quant.rs:864-873). Every lane of the half-wave must call this.
__device__ __forceinline__ void quant_lane(float v, bool valid, int8_t* q, float* s, uint16_t* h) {
    float m = fmaxf(0.0f, fabsf(v));
    m = group_max32(m);
    float d = div_rn(m, 127.0f);
    float inv = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
    if (valid) {
        *q = q8_round(v * inv);
        if ((threadIdx.x & 31) == 0) {
            *s = d;
            *h = f16_bits(d);
        }
    }
}

// Position of block t in a chain-major row of nb blocks (nb % 4 == 0): the
// blocks of the reference's partial sum 0 (t = 0, 4, 8, ..), then those of
// sums 1, 2 and 3, each in block order.
__device__ __forceinline__ uint32_t cm_block(uint32_t t, uint32_t nb) { return (t & 3) * (nb >> 2) + (t >> 2); }

__device__ __forceinline__ uint32_t win_slot(const DevWindow& w, uint32_t n_shared, uint32_t i) {
    return i < n_shared ? w.shared_start + i : w.att_start + (i - n_shared);
}

// Up to three matrices with the same K projected in one launch (q/k/v, or
// gate/up): the grid is the concatenation of their column-tile ranges.
struct MatSet {
    const int8_t* q[3];
    const void* s[3];
    float* y[3];
    uint32_t n[3];
    uint32_t ld[3];
    uint32_t tile_end[3];  // cumulative tile counts
    int count;
};

// A scale as loaded: f32 bits, or f16 bits that are widened only where the
// value is used (widening right after the load would make its wait immediate).
__device__ __forceinline__ uint32_t scale_bits(bool f16, const void* p, size_t i) {
    return f16 ? (uint32_t)((const uint16_t*)p)[i] : f2u(((const float*)p)[i]);
}
__device__ __forceinline__ float scale_value(bool f16, uint32_t bits) {
    return f16 ? f16w((uint16_t)bits) : u2f(bits);
}

// The four-partial Q8_0 GEMM (gemm.hip) over a matrix set, rows >= 8.
hipError_t launch_gemm_q8(hipStream_t st, int sem, const MatSet& ms, size_t k, QuantAct x, size_t rows,
                          int32_t* dbg);

// The chunk pipeline shared by both GEMM kernels. At chunk c, the register
// stage (c + 1) % NS holds chunk c + 1 and LDS buffer c & 1 holds chunk c.
// The chunk count is padded to a multiple of NS and every load and store is
// unconditional (loads clamp to the last chunk, compute skips blocks past
// the end), so all paths issue the same loads and each wait covers only the
// chunk about to be stored.
template <int NS, typename Stage, typename Load, typename Store, typename Compute>
__device__ __forceinline__ void gemm_pipeline(uint32_t nchunks, Load&& gload, Store&& lstore, Compute&& compute) {
    static_assert(NS % 2 == 0, "the LDS buffer parity follows the register stage");
    Stage st[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) gload(st[s], s);
    lstore(st[0], 0);
    gload(st[0], NS);
    __syncthreads();
    const uint32_t steps = (nchunks + NS - 1) / NS * NS;
    for (uint32_t c0 = 0; c0 < steps; c0 += NS) {
#pragma unroll
        for (int u = 0; u < NS; u++) {
            compute(u & 1, c0 + u);
            lstore(st[(u + 1) % NS], (u + 1) & 1);
            gload(st[(u + 1) % NS], c0 + u + 1 + NS);
            __syncthreads();
        }
    }
}

}  // namespace kr

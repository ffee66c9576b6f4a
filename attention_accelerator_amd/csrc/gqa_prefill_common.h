// gqa_prefill_common.h -- pieces shared by the chunked-prefill attention kernel
// (gqa_prefill.hip) and the multi-token decode kernels (gqa_multitoken.hip): the chunk's
// start check, cache addressing, the swizzled LDS row layout that K/V copies land in, and
// the three-part split of the softmax probabilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gqa_device.h"
#include "gqa_internal.h"

namespace gqa {

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kRowB = 256;                  // LDS bytes per K/V row
constexpr uint32_t kPermHi = 0x07060302u;   // byte selector: the high halves of two dwords

__device__ __forceinline__ bool prefill_start_ok(const PrefillArgs& a, int st) {
    return st >= 0 && st <= a.capacity - a.n_new;
}

// Element offset of cache row (b, h, p); -1 for a paged cache whose block id for p is
// outside the pool.
__device__ __forceinline__ int64_t cache_elem(const PrefillArgs& a, int b, int h, int64_t p) {
    if (a.block_table) {
        const int pid = a.block_table[static_cast<int64_t>(b) * a.max_blocks + p / 16];
        if (pid < 0 || pid >= a.n_blocks) return -1;
        return static_cast<int64_t>(pid) * a.kv_batch_stride + static_cast<int64_t>(h) * a.kv_head_stride +
               (p % 16) * a.kv_pos_stride;
    }
    return static_cast<int64_t>(b) * a.kv_batch_stride + static_cast<int64_t>(h) * a.kv_head_stride +
           p * a.kv_pos_stride;
}

// K/V rows copied HBM -> LDS land as 16 16-byte chunks per 256-byte row; chunk c of row r
// sits at position c ^ pf_swz(r & 15), so that 16-row operand reads and the V^T transpose
// reads hit 64 distinct banks per pass.
__device__ __forceinline__ int pf_swz(int row) {
    const int r = row & 15;
    return (2 * r + (r >> 3)) & 15;
}

// 8 K values of row `row`, bytes [16 chunk, 16 chunk + 16) of the plane at `plane`.
__device__ __forceinline__ bf16x8_t pf_k_chunk(const uint8_t* plane, int row, int chunk) {
    return *reinterpret_cast<const bf16x8_t*>(plane + row * kRowB + 16 * (chunk ^ pf_swz(row)));
}

// Offset within a V plane of lane `lane`'s transpose read (ds_read_b64_tr_b16) for dim tile
// dt, keys 0..15 of the plane: lane (g, a) addresses row 4g + a/4, dims 16dt + 4(a%4) .. +3
// (the reads 16 rows further are this offset + 4096).
__device__ __forceinline__ uint32_t vt_tr_offset(int dt, int lane) {
    const int g = lane >> 4;
    const int a = lane & 15;
    const int row = 4 * g + (a >> 2);
    const int chunk = 2 * dt + ((a & 3) >> 1);
    return row * kRowB + 16 * (chunk ^ pf_swz(row)) + (a & 1) * 8;
}

// Upper 16 bits of two floats packed as BF16 codes (truncation; used for exact splits).
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), kPermHi);
}

// p = 2^(s - m) of key tile kt (0 for masked keys), summed into lsum, split by truncation
// into three BF16 parts packed as the P^T B operand: ph[part][window][dword].
__device__ __forceinline__ void pf_probs_tile(const f32x4_t& s, float m, float& lsum, uint32_t (&ph)[3][2][4],
                                              int kt) {
    float p[4], r1[4], r2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // v_exp_f32: 2^x, 0 for -inf (masked keys); results below 2^-126 flush to 0, far
        // below anything the BF16 output can see.
        p[i] = __builtin_amdgcn_exp2f(s[i] - m);
        lsum += p[i];
        r1[i] = p[i] - __uint_as_float(__float_as_uint(p[i]) & 0xffff0000u);
        r2[i] = r1[i] - __uint_as_float(__float_as_uint(r1[i]) & 0xffff0000u);
    }
    const int w = kt >> 1, d0 = (kt & 1) * 2;
    ph[0][w][d0] = pack_hi16(p[0], p[1]);
    ph[0][w][d0 + 1] = pack_hi16(p[2], p[3]);
    ph[1][w][d0] = pack_hi16(r1[0], r1[1]);
    ph[1][w][d0 + 1] = pack_hi16(r1[2], r1[3]);
    ph[2][w][d0] = pack_hi16(r2[0], r2[1]);
    ph[2][w][d0 + 1] = pack_hi16(r2[2], r2[3]);
}

}  // namespace gqa

// gqa_prefill.hip -- chunked prefill (multi-query GQA) on MFMA for gfx950, and the KV
// append with RoPE on insert.
//
// The reference core computes one query token per start (gqa_controller.v:140-277;
// golden pyfiles/gen_gqa_wrapper_vectors.py:121-139).  A prefill chunk is that step for
// T consecutive tokens of a sequence: token t sits at position start+t and attends to
// keys p <= start+t (the causal half of gqa_attention_wrapper.v:279), where keys
// p < start are cache rows as stored (post-RoPE) and keys start..start+T-1 are the
// chunk's own K/V rows, rotated at their positions in double and not re-rounded, as
// the golden rotates K (gen_gqa_wrapper_vectors.py:124-126).
//
// kv_append_kernel writes the chunk's K rows (rotated, rounded double -> f32 -> BF16,
// pyfiles/gqa_reference.py:15-19) and V rows into the cache, and the second and third
// BF16 parts of each rotated K row into the workspace, so that the cache row plus
// those two parts carry the rotated value to ~24 bits.
//
// prefill_attn_kernel: one workgroup of 8 waves per (sequence, KV head, 32 query
// positions); wave w computes Q head 4*kv_head + (w & 3) for 16 positions.  The K/V
// rows of each 64-key block are copied once per workgroup into LDS and used by all 4
// heads of the group and all 32 positions (gqa_kv_broadcast.v:38-59 at block scale).
// K runs one block ahead of V, so that each wave forms block j's probabilities while its
// MFMAs form block j+1's scores, then accumulates block j's V^T P^T.
//
//  * Scores S^T = K Q^T with v_mfma_f32_16x16x32_bf16: A = 16 keys x 32 dims of K from
//    LDS (row = key), B = Q^T (column = query) held in registers.  Q is rotated and
//    scaled by scale*log2(e) in double and split into three BF16 parts, so the exact
//    bf16 x bf16 products carry ~24 bits of Q; for blocks with chunk keys the second and
//    third parts of K add the (k2,q1), (k2,q2), (k3,q1) products.  Lane (g, n) ends with
//    the scores of keys 4g+i (i = 0..3) of each 16-key tile for query n.
//  * Online softmax per query with an integer-valued running max (every rescale is an
//    exact power of two), p = exp2(s - m) in fp32, masked keys p = 0 exactly.
//  * O^T += V^T P^T with the same MFMA: A = 16 dims x 32 keys of V^T from LDS, B = P^T.
//    The lane already holds P for keys {4g+i} of tiles 2w and 2w+1, which is its B
//    operand for the 32-key window w if V^T stores each window's keys in that order
//    (slot 8g+4h+i <-> key 16h+4g+i).  P is split into three BF16 parts (~24 bits).
//    Each block's fp32 product is added to an fp64 accumulator, so accumulation over
//    thousands of keys adds no fp32 rounding.
//  * O / l, rounded double -> f32 -> BF16, written in Q-head order.
//
// Chunks of at most 16 new tokens take the multi-token decode path instead
// (gqa_multitoken.hip), which shares this file's LDS row layout and probability split
// (gqa_prefill_common.h).
#include "gqa_device.h"
#include "gqa_internal.h"
#include "gqa_prefill_common.h"

namespace gqa {

namespace {

constexpr int kPfPos = 32;                 // query positions per workgroup
constexpr int kPfWaves = 8;                // 4 Q heads x 2 tiles of 16 positions
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfBlk = 64;                 // keys per K/V block

}  // namespace

// The second and third BF16 parts of every rotated new K row, then one zero row (the parts
// of a cached key, which the attention kernel copies for keys before the chunk).
size_t prefill_split_bytes(int32_t batch, int32_t n_new) {
    return (2ull * static_cast<size_t>(batch) * static_cast<size_t>(n_new) * kHkv + 1) * kD * sizeof(uint16_t);
}

// ---------------------------------------------------------------------------------
// KV append: one wave per new (sequence, token); lane i computes the angle of frequency i
// at position start+t once (pyfiles/gen_gqa_wrapper_vectors.py:30-31) and rotates the
// pair (i, i+64) of all 8 KV heads' rows in double (:25-35).  All 8 heads' rows are
// requested before any is written, so a wave waits for memory once.
__global__ __launch_bounds__(256) void kv_append_kernel(PrefillArgs a) {
    const int64_t bt = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);   // b * T + t
    const int lane = threadIdx.x & (kWave - 1);
    if (a.k_split && blockIdx.x == 0 && threadIdx.x < kD / 2) {
        uint32_t* zero_row = reinterpret_cast<uint32_t*>(
            a.k_split + 2 * static_cast<int64_t>(a.batch) * a.n_new * kHkv * kD);
        zero_row[threadIdx.x] = 0u;
    }
    if (blockIdx.x == 0) rs_clear(a, threadIdx.x);
    if (bt >= static_cast<int64_t>(a.batch) * a.n_new) return;
    const int t = static_cast<int>(bt % a.n_new);
    const int b = static_cast<int>(bt / a.n_new);
    const int st = a.start[b];
    if (!prefill_start_ok(a, st)) return;
    const int64_t pos = static_cast<int64_t>(st) + t;
    const int64_t n_rows = static_cast<int64_t>(a.batch) * a.n_new * kHkv;
    const bool rope = (a.flags & 2u) != 0;
    uint16_t kx[kHkv], ky[kHkv], vx[kHkv], vy[kHkv];
    int64_t ce[kHkv];
#pragma unroll
    for (int kvh = 0; kvh < kHkv; ++kvh) {
        const int64_t row = bt * kHkv + kvh;
        kx[kvh] = a.k_new[row * kD + lane];
        ky[kvh] = a.k_new[row * kD + lane + kPairs];
        vx[kvh] = a.v_new[row * kD + lane];
        vy[kvh] = a.v_new[row * kD + lane + kPairs];
        ce[kvh] = cache_elem(a, b, kvh, pos);
    }
    double sn = 0.0, cs = 1.0;
    const bool any_rope = (a.flags & 3u) != 0;        // the rescore rotates Q with these too
    if (any_rope) rope_sincos(pos, a.rope.inv_freq[lane], sn, cs);
    if (a.rs_hdr) {
        if (lane < kHq) a.rs_done[bt * kHq + lane] = 0u;
        if (any_rope) a.rs_cs[bt * kPairs + lane] = make_double2(cs, sn);
    }
#pragma unroll
    for (int kvh = 0; kvh < kHkv; ++kvh) {
        const int64_t row = bt * kHkv + kvh;
        const double x = bf16_to_f32(kx[kvh]);
        const double y = bf16_to_f32(ky[kvh]);
        double xr = x, yr = y;
        if (rope) {
            xr = x * cs - y * sn;
            yr = x * sn + y * cs;
        }
        const uint16_t hx = bf16_of(xr), hy = bf16_of(yr);
        if (ce[kvh] >= 0) {
            uint16_t* kdst = a.k + ce[kvh];
            uint16_t* vdst = a.v + ce[kvh];
            kdst[lane] = hx;
            kdst[lane + kPairs] = hy;
            vdst[lane] = vx[kvh];
            vdst[lane + kPairs] = vy[kvh];
        }
        if (a.k_split) {
            const double rx = xr - f64_of_bf16(hx), ry = yr - f64_of_bf16(hy);
            const uint16_t mx = bf16_of(rx), my = bf16_of(ry);
            uint16_t* mid = a.k_split + row * kD;
            uint16_t* lo = a.k_split + (n_rows + row) * kD;
            mid[lane] = mx;
            mid[lane + kPairs] = my;
            lo[lane] = bf16_of(rx - f64_of_bf16(mx));
            lo[lane + kPairs] = bf16_of(ry - f64_of_bf16(my));
        }
    }
}

hipError_t launch_kv_append(const PrefillArgs& a, hipStream_t stream) {
    const int64_t n_tok = static_cast<int64_t>(a.batch) * a.n_new;
    if (n_tok == 0) return hipSuccess;
    hipLaunchKernelGGL(kv_append_kernel, dim3(static_cast<unsigned>((n_tok + 3) / 4)), dim3(256), 0,
                       stream, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Attention.

// LDS: eight 16 KB planes of 64 rows x 256 B -- K of buffers 0 and 1, V of buffers 0 and 1,
// then the second and third BF16 parts of chunk keys for buffers 0 and 1 (128 KB in all).
// K runs one block ahead of V: while block j's probabilities are formed and its V^T P^T
// accumulated, block j+1's scores are formed from the other K buffer.  Rows are copied from
// HBM straight into LDS (global_load_lds_dwordx4: lane l of an instruction writes bytes
// [16l, 16l + 16) of a 1 KB stretch = 4 rows), so a row's 16 16-byte chunks are placed by
// choosing which chunk each lane fetches: chunk c of row r sits at position c ^ pf_swz(r & 15).
// With that swizzle the K operand reads (16 rows, one chunk) and the V^T transpose reads
// (16 rows, two chunks) hit 64 distinct banks per pass, and because it depends on r & 15 only,
// the rows 16 apart that one lane reads differ by a constant offset.
constexpr int kPlaneB = kPfBlk * kRowB;     // 16 KB per plane
constexpr int kOffK = 0;                    // + buffer * kPlaneB
constexpr int kOffV = 2 * kPlaneB;
constexpr int kOffK2 = 4 * kPlaneB;
constexpr int kOffK3 = 6 * kPlaneB;
constexpr int kLdsB = 8 * kPlaneB;

typedef __attribute__((address_space(3))) void lds_void_t;

// Wave w of the workgroup copies rows 8w .. 8w+7 of a plane (two 4-row instructions).
// Rows past the keys this workgroup needs repeat its last key.
__device__ __forceinline__ int pf_copy_row(int wave, int ii, int lane) { return 4 * (2 * wave + ii) + (lane >> 4); }

// Request the K rows of block blk into K buffer `buf`, and for a block holding chunk keys the
// second and third parts of its rows (a cached key's parts come from the zero row).  For a
// block whose 64 keys all exist the addresses are the block's first row (uniform) plus the
// lane's 32-bit offset `loff` (pf_copy_offsets).
__device__ __forceinline__ void pf_issue_k(const PrefillArgs& a, const char* kbase, int b, int kvh, int st,
                                           int blk, int n_keys, bool has_new, const uint32_t (&loff)[2],
                                           uint8_t* lds, int buf, int wave, int lane) {
    const int64_t row_bytes = a.kv_pos_stride * 2;
    const int64_t n_rows = static_cast<int64_t>(a.batch) * a.n_new * kHkv;
    const int key0 = blk * kPfBlk;
    if (!has_new && key0 + kPfBlk <= n_keys) {
        // the common block: cached keys only, all 64 rows exist (a uniform branch, so no
        // per-lane address arithmetic beyond the lane's fixed offset)
        const char* brow = kbase + static_cast<int64_t>(key0) * row_bytes;
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
            __builtin_amdgcn_global_load_lds(brow + loff[ii],
                                             (lds_void_t*)(lds + kOffK + buf * kPlaneB + (2 * wave + ii) * 1024), 16, 0, 0);
        return;
    }
    const bool full = key0 + kPfBlk <= n_keys;
    const char* brow = kbase + static_cast<int64_t>(key0) * row_bytes;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int r = pf_copy_row(wave, ii, lane);
        const int c = (lane & 15) ^ pf_swz(r);
        const int key = min(key0 + r, n_keys - 1);
        const int stretch = buf * kPlaneB + (2 * wave + ii) * 1024;
        const char* src = full ? brow + loff[ii] : kbase + static_cast<int64_t>(key) * row_bytes + 16 * c;
        __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(lds + kOffK + stretch), 16, 0, 0);
        if (has_new) {
            const int u = key - st;          // chunk row of this key (< 0: a cached key)
            const int64_t prow = u < 0 ? 2 * n_rows : (static_cast<int64_t>(b) * a.n_new + u) * kHkv + kvh;
            const int64_t lrow = u < 0 ? 2 * n_rows : n_rows + prow;
            const char* p1 = reinterpret_cast<const char*>(a.k_split + prow * kD) + 16 * c;
            const char* p2 = reinterpret_cast<const char*>(a.k_split + lrow * kD) + 16 * c;
            __builtin_amdgcn_global_load_lds(p1, (lds_void_t*)(lds + kOffK2 + stretch), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(p2, (lds_void_t*)(lds + kOffK3 + stretch), 16, 0, 0);
        }
    }
}

// Request the V rows of block blk into V buffer `buf` (addresses as in pf_issue_k).
__device__ __forceinline__ void pf_issue_v(const PrefillArgs& a, const char* vbase, int blk, int n_keys,
                                           const uint32_t (&loff)[2], uint8_t* lds, int buf, int wave, int lane) {
    const int64_t row_bytes = a.kv_pos_stride * 2;
    const int key0 = blk * kPfBlk;
    const bool full = key0 + kPfBlk <= n_keys;
    const char* brow = vbase + static_cast<int64_t>(key0) * row_bytes;
    if (full) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
            __builtin_amdgcn_global_load_lds(brow + loff[ii],
                                             (lds_void_t*)(lds + kOffV + buf * kPlaneB + (2 * wave + ii) * 1024), 16, 0, 0);
        return;
    }
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int r = pf_copy_row(wave, ii, lane);
        const int c = (lane & 15) ^ pf_swz(r);
        const int key = min(key0 + r, n_keys - 1);
        const int stretch = buf * kPlaneB + (2 * wave + ii) * 1024;
        const char* src = full ? brow + loff[ii] : vbase + static_cast<int64_t>(key) * row_bytes + 16 * c;
        __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(lds + kOffV + stretch), 16, 0, 0);
    }
}

// The lane's byte offset from a block's first row for its two copy instructions (below 2^32:
// the ABI keeps (capacity + 64) rows of a (sequence, KV head) under 4 GiB).
__device__ __forceinline__ void pf_copy_offsets(const PrefillArgs& a, int wave, int lane, uint32_t (&loff)[2]) {
    const uint32_t row_bytes = static_cast<uint32_t>(a.kv_pos_stride * 2);
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int r = pf_copy_row(wave, ii, lane);
        loff[ii] = static_cast<uint32_t>(r) * row_bytes + 16u * static_cast<uint32_t>((lane & 15) ^ pf_swz(r));
    }
}

// One 32-dim slice (dims 32q .. 32q+31) of the scores S^T[key][query] of one 16-query tile
// over the block's 4 key tiles: the 3 BF16 parts of Q against the cache row, and for chunk
// keys the (k2,q1), (k2,q2), (k3,q1) products.
template <bool kNew>
__device__ __forceinline__ void pf_qk_slice(const uint8_t* kplane, const bf16x8_t (&qop)[3][4], int q, int n,
                                            int g, f32x4_t (&sacc)[4]) {
    bf16x8_t ak[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k_chunk(kplane, 16 * kt + n, 4 * q + g);
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
            sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[kt], qop[s][q], sacc[kt], 0, 0, 0);
    if (kNew) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k_chunk(kplane + (kOffK2 - kOffK), 16 * kt + n, 4 * q + g);
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
                sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[kt], qop[s][q], sacc[kt], 0, 0, 0);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k_chunk(kplane + (kOffK3 - kOffK), 16 * kt + n, 4 * q + g);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
            sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[kt], qop[0][q], sacc[kt], 0, 0, 0);
    }
}

// Per-tile softmax state: the running max (integer-valued, log2 units), sum and O (fp64,
// lane (g, n): O^T[16dt + 4g + i][query n]).
struct PfTile {
    double o64[8][4];
    double l64;
    float m_run;
};

// Running max after a block: masks keys past each query on diagonal blocks, then returns
// ceil(block max) where that exceeds the running max m (integer-valued, so every rescale is an
// exact power of two), else m.  The two cross-row steps are gfx950 lane swaps (rows 16 and 32
// lanes apart), not LDS permutes.
__device__ __forceinline__ float pf_next_max(f32x4_t (&sacc)[4], bool diag, int key0, int g, int pos_n, float m) {
    if (diag) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (key0 + 16 * kt + 4 * g + i > pos_n) sacc[kt][i] = -INFINITY;
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) bmax = fmaxf(bmax, sacc[kt][i]);
    const auto x16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(bmax), __float_as_uint(bmax), false, false);
    bmax = fmaxf(__uint_as_float(x16[0]), __uint_as_float(x16[1]));
    const auto x32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(bmax), __float_as_uint(bmax), false, false);
    bmax = fmaxf(__uint_as_float(x32[0]), __uint_as_float(x32[1]));
    return bmax > m ? ceilf(bmax) : m;
}

// Moves O and l to the running max m_new (exact power-of-two scaling).
__device__ __forceinline__ void pf_rescale(PfTile& t, float m_new) {
    if (__ballot(m_new != t.m_run)) {
        const int shift = (t.m_run == -INFINITY) ? 0 : static_cast<int>(t.m_run - m_new);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) t.o64[dt][i] = ldexp(t.o64[dt][i], shift);
        t.l64 = ldexp(t.l64, shift);
        t.m_run = m_new;
    }
}

// V^T operands of one 16-dim tile dt for both 32-key windows: lane (g, m) gets keys
// 32w + 4g + i (slots 0..3) and 32w + 16 + 4g + i (slots 4..7) of dim 16dt + m, through
// transpose reads (ds_read_b64_tr_b16: lane i of a 16-lane group receives element i%4 of the
// 8 bytes addressed by lane 4j + i/4, j = 0..3).  Supplying lane a addresses row
// 32w + 4g + a/4 (+16), dims 16dt + 4(a%4) .. +3; `addr` is that address for w = 0 without
// the +16, and the other three rows are 16, 32 and 48 rows further.
//
// The reads are issued from inline assembly and waited for by pf_vt_wait: the compiler
// treats every transpose read as possibly reading LDS that an outstanding copy writes and
// would wait for all of them (the next block's copies included) before the first one.  The
// copies that fill the buffer read here completed before the barrier that opened this block.
struct VtPair {
    short4_t r[2][2];   // [window][half]
};

__device__ __forceinline__ VtPair pf_vt_issue(uint32_t addr) {
    VtPair v;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v.r[0][0]) : "v"(addr));
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:4096" : "=v"(v.r[0][1]) : "v"(addr));
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:8192" : "=v"(v.r[1][0]) : "v"(addr));
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:12288" : "=v"(v.r[1][1]) : "v"(addr));
    return v;
}

// Waits for every outstanding LDS read (lgkmcnt(0)); tied to the operands so that their uses
// stay behind it.
__device__ __forceinline__ void pf_vt_wait(VtPair& v0, VtPair& v1) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v0.r[0][0]), "+v"(v0.r[0][1]), "+v"(v0.r[1][0]), "+v"(v0.r[1][1]), "+v"(v1.r[0][0]),
                   "+v"(v1.r[0][1]), "+v"(v1.r[1][0]), "+v"(v1.r[1][1]));
}

__device__ __forceinline__ bf16x8_t pf_vt_operand(const VtPair& v, int w) {
    union {
        short4_t h[2];
        bf16x8_t v;
    } u;
    u.h[0] = v.r[w][0];
    u.h[1] = v.r[w][1];
    return u.v;
}

// Per-lane LDS address of the transpose reads of dim tile dt (V buffer 0, window 0).
__device__ __forceinline__ uint32_t pf_vt_addr(uint32_t lds_base, int dt, int lane) {
    return lds_base + kOffV + vt_tr_offset(dt, lane);
}

// O^T[dim][query] += the block's V^T P^T: per 16-dim tile, V^T (transpose reads) against the
// three P parts of both 32-key windows in fp32, then added into the fp64 O; two tiles at a
// time, the next two tiles' operands requested before the current two's products.
__device__ __forceinline__ void pf_pv(const uint32_t (&vaddr)[8], uint32_t voff, const uint32_t (&ph)[3][2][4],
                                      PfTile& t) {
    bf16x8_t pb[2][3];
#pragma unroll
    for (int w = 0; w < 2; ++w)
#pragma unroll
        for (int s = 0; s < 3; ++s) pb[w][s] = as_bf16x8(make_uint4(ph[s][w][0], ph[s][w][1], ph[s][w][2], ph[s][w][3]));
    VtPair cur[2];
    cur[0] = pf_vt_issue(vaddr[0] + voff);
    cur[1] = pf_vt_issue(vaddr[1] + voff);
#pragma unroll
    for (int d0 = 0; d0 < 8; d0 += 2) {
        pf_vt_wait(cur[0], cur[1]);
        VtPair nxt[2];
        if (d0 + 2 < 8) {
            nxt[0] = pf_vt_issue(vaddr[d0 + 2] + voff);
            nxt[1] = pf_vt_issue(vaddr[d0 + 3] + voff);
        }
        f32x4_t oacc[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) oacc[e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const bf16x8_t av = pf_vt_operand(cur[e], w);
#pragma unroll
                for (int s = 0; s < 3; ++s)
                    oacc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[w][s], oacc[e], 0, 0, 0);
            }
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) t.o64[d0 + e][i] += static_cast<double>(oacc[e][i]);
        if (d0 + 2 < 8) {
            cur[0] = nxt[0];
            cur[1] = nxt[1];
        }
    }
}

// Probabilities of the current block (scores `scur`, running max already grown) interleaved
// with the scores of the next block from K buffer `kplane` (kNext: there is one; kNew: it
// holds chunk keys).
template <bool kNext, bool kNew>
__device__ __forceinline__ void pf_probs_and_next(const f32x4_t (&scur)[4], const uint8_t* kplane,
                                                  const bf16x8_t (&qop)[3][4], int n, int g, PfTile& t,
                                                  uint32_t (&ph)[3][2][4], f32x4_t (&snext)[4]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) snext[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (kNext) pf_qk_slice<kNew>(kplane, qop, q, n, g, snext);
        pf_probs_tile(scur[q], t.m_run, lsum, ph, q);
    }
    t.l64 += static_cast<double>(lsum);
}

__global__ __launch_bounds__(kPfThreads) void prefill_attn_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsB];

    // Workgroup -> (sequence, KV head, query block).  Workgroups are dealt to the 8 XCDs
    // round-robin; when the (sequence, KV head) pairs divide evenly, all query blocks of
    // a pair go to one XCD so that its K/V blocks are shared in that XCD's L2.
    const int n_pairs = a.batch * kHkv;
    const int id = blockIdx.x;
    int pair, qb;
    if (n_pairs % 8 == 0) {
        const int k = id >> 3;
        qb = k % a.n_qblk;
        pair = (k / a.n_qblk) * 8 + (id & 7);
    } else {
        pair = id / a.n_qblk;
        qb = id % a.n_qblk;
    }
    const int b = pair / kHkv;
    const int kvh = pair % kHkv;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & (kWave - 1);
    const int n = lane & 15;
    const int g = lane >> 4;
    const int hq = kvh * kGroup + (wave & 3);
    const int pt = wave >> 2;
    const int T = a.n_new;
    const int t_wave0 = qb * kPfPos + pt * 16;
    const int tq = t_wave0 + n;
    const bool q_ok = tq < T;
    const int st = a.start[b];

    if (!prefill_start_ok(a, st)) {
        if (q_ok && g == 0) {
            uint4* o = reinterpret_cast<uint4*>(a.out + ((static_cast<int64_t>(b) * T + tq) * kHq + hq) * kD);
            for (int i = 0; i < kD / 8; ++i) o[i] = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
        }
        return;
    }

    // Every wave runs every block of the workgroup; a block past the keys of this wave's
    // queries is masked for all of them (block 0 always holds a valid key, so the running
    // max is finite from the first block on).  Waves past the last query compute the last
    // query and write nothing.
    const int tq_c = min(tq, T - 1);
    const int pos_n = st + tq_c;            // this lane's query position
    const int n_keys = st + min(T, qb * kPfPos + kPfPos);
    const int n_blk = (n_keys + kPfBlk - 1) / kPfBlk;
    const int64_t head_elem = static_cast<int64_t>(b) * a.kv_batch_stride +
                              static_cast<int64_t>(kvh) * a.kv_head_stride;
    const char* kbase = reinterpret_cast<const char*>(a.k + head_elem);
    const char* vbase = reinterpret_cast<const char*>(a.v + head_elem);
    auto blk_new = [&](int blk) { return blk * kPfBlk + kPfBlk - 1 >= st; };
    auto blk_diag = [&](int blk) { return blk * kPfBlk + kPfBlk - 1 > st + t_wave0; };

    // K of blocks 0 and 1 and V of block 0 are requested before the Q operands are formed.
    uint32_t loff[2];
    pf_copy_offsets(a, wave, lane, loff);
    pf_issue_k(a, kbase, b, kvh, st, 0, n_keys, blk_new(0), loff, lds, 0, wave, lane);
    pf_issue_v(a, vbase, 0, n_keys, loff, lds, 0, wave, lane);
    if (n_blk > 1) pf_issue_k(a, kbase, b, kvh, st, 1, n_keys, blk_new(1), loff, lds, 1, wave, lane);

    // Q operands: query n = this lane's column, dims 32kb + 8g + j, three BF16 parts.
    bf16x8_t qop[3][4];
    {
        const uint16_t* qrow = a.q + ((static_cast<int64_t>(b) * T + tq_c) * kHq + hq) * kD;
        double qv[4][8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = 32 * kb + 8 * g + j;
                const double x = bf16_to_f32(qrow[d]);
                const double y = bf16_to_f32(qrow[d + kPairs]);
                double xr = x, yr = y;
                if (a.flags & 1u) rope_pair(x, y, pos_n, a.rope.inv_freq[d], xr, yr);
                qv[kb][j] = xr * a.qk_scale_log2;
                qv[kb + 2][j] = yr * a.qk_scale_log2;
            }
        }
#pragma unroll
        for (int s = 0; s < 3; ++s)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                uint16_t h8[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) h8[j] = split3(qv[kb][j], s);
                // Pin the operand: without this the compiler re-derives it from the double
                // rows inside the block loop (~600 extra VALU per block) to save registers.
                union {
                    bf16x8_t v;
                    uint32_t w[4];
                } u;
                u.v = pack8(h8);
                asm volatile("" : "+v"(u.w[0]), "+v"(u.w[1]), "+v"(u.w[2]), "+v"(u.w[3]));
                qop[s][kb] = u.v;
            }
    }

    const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(lds)));
    uint32_t vaddr[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) vaddr[dt] = pf_vt_addr(lds_base, dt, lane);

    PfTile tl;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) tl.o64[dt][i] = 0.0;
    tl.l64 = 0.0;
    tl.m_run = -INFINITY;

    // Block 0's scores.  The barrier after them frees K buffer 0 for block 2.
    __builtin_amdgcn_s_waitcnt(0x0F70);    // vmcnt(0)
    __syncthreads();
    f32x4_t scur[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) scur[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (blk_new(0)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) pf_qk_slice<true>(lds + kOffK, qop, q, n, g, scur);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) pf_qk_slice<false>(lds + kOffK, qop, q, n, g, scur);
    }
    pf_rescale(tl, pf_next_max(scur, blk_diag(0), 0, g, pos_n, tl.m_run));
    __syncthreads();

    for (int blk = 0; blk < n_blk; ++blk) {
        // Resident: K of block blk+1 (K buffer (blk+1)&1) and V of block blk (V buffer blk&1).
        // Free: K buffer blk&1 (block blk, scored in the previous step) and V buffer
        // (blk+1)&1 (block blk-1).
        if (blk + 2 < n_blk)
            pf_issue_k(a, kbase, b, kvh, st, blk + 2, n_keys, blk_new(blk + 2), loff, lds, blk & 1, wave, lane);
        if (blk + 1 < n_blk) pf_issue_v(a, vbase, blk + 1, n_keys, loff, lds, (blk + 1) & 1, wave, lane);

        uint32_t ph[3][2][4];
        f32x4_t snext[4];
        const uint8_t* knext = lds + kOffK + ((blk + 1) & 1) * kPlaneB;
        // The two waves of a SIMD run the same steps; the one in this MFMA + VALU mix gets
        // issue priority over the other's V^T P^T (5 % faster than equal priorities).
        __builtin_amdgcn_s_setprio(1);
        if (blk + 1 >= n_blk)
            pf_probs_and_next<false, false>(scur, knext, qop, n, g, tl, ph, snext);
        else if (blk_new(blk + 1))
            pf_probs_and_next<true, true>(scur, knext, qop, n, g, tl, ph, snext);
        else
            pf_probs_and_next<true, false>(scur, knext, qop, n, g, tl, ph, snext);
        __builtin_amdgcn_s_setprio(0);

        // The next block's running max is found before this block's V^T P^T (which still
        // accumulates at the current max); O and l move to it afterwards.
        float m_next = tl.m_run;
        if (blk + 1 < n_blk) m_next = pf_next_max(snext, blk_diag(blk + 1), (blk + 1) * kPfBlk, g, pos_n, tl.m_run);

        pf_pv(vaddr, (blk & 1) * kPlaneB, ph, tl);

        pf_rescale(tl, m_next);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) scur[kt] = snext[kt];
        // This wave's copies into LDS are complete; after the barrier every wave's are, and
        // every wave is done with the buffers the next step's copies go to.
        __builtin_amdgcn_s_waitcnt(0x0F70);    // vmcnt(0)
        __syncthreads();
    }

    double l = tl.l64 + __shfl_xor(tl.l64, 16);
    l += __shfl_xor(l, 32);
    // The row of query n (lanes n, n+16, n+32, n+48 hold dims 16dt + 4g ..): its smallest
    // magnitude against its rms decides whether the row is rescored in fp64.
    double x[8][4], ss = 0.0, mn = INFINITY;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[dt][i] = tl.o64[dt][i] / l;
            ss = fma(x[dt][i], x[dt][i], ss);
            mn = fmin(mn, fabs(x[dt][i]));
        }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    mn = fmin(mn, __shfl_xor(mn, 16));
    mn = fmin(mn, __shfl_xor(mn, 32));
    if (!q_ok) return;
    if (g == 0 && a.rs_hdr && mn * mn * kD < kRsFlagRatio2 * ss)
        rs_append(a, static_cast<uint32_t>((static_cast<int64_t>(b) * T + tq) * kHq + hq));
    {
        uint16_t* orow = a.out + ((static_cast<int64_t>(b) * T + tq) * kHq + hq) * kD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            uint2 pk;
            pk.x = f32_to_bf16_rne(static_cast<float>(x[dt][0])) |
                   (static_cast<uint32_t>(f32_to_bf16_rne(static_cast<float>(x[dt][1]))) << 16);
            pk.y = f32_to_bf16_rne(static_cast<float>(x[dt][2])) |
                   (static_cast<uint32_t>(f32_to_bf16_rne(static_cast<float>(x[dt][3]))) << 16);
            *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * g) = pk;
        }
    }
}

hipError_t launch_prefill_attention(const PrefillArgs& a, hipStream_t stream) {
    const int64_t n_wg = static_cast<int64_t>(a.batch) * kHkv * a.n_qblk;
    if (n_wg == 0) return hipSuccess;
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(static_cast<unsigned>(n_wg)), dim3(kPfThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace gqa

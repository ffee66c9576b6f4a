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
// Four launches, then the fp64 rescore of flagged rows (gqa_decode.hip):
//
// kv_append_kernel writes the chunk's K rows (rotated, rounded double -> f32 -> BF16,
// pyfiles/gqa_reference.py:15-19) and V rows into the cache, and the rotated K rows in fp32
// (24 bits, not rounded to BF16) into the workspace.
//
// prefill_stage_kernel copies the K/V rows the attention reads -- cache rows before the
// chunk, the chunk's rows -- into fp16 planes in the workspace, one power-of-two scale per
// (sequence, KV head, block of 64 positions) putting the block's largest magnitude in
// [2^14, 2^15).  A BF16 value has an 8-bit significand, so it converts exactly unless it
// lies more than ~2^31 below that largest magnitude; a chunk key's fp32 value becomes two
// fp16 parts (leading + trailing, ~22 bits).  A block holding a non-finite value, a scale
// outside the fp32 range the attention kernel uses, or a row more than 2^12 below the
// block's largest magnitude is marked, and the attention kernel hands all rows that read
// it to the fp64 rescore.  It also leaves each block's K pair-group norm and |V| maxima.
//
// prefill_stat_reduce_kernel folds those block maxima into the maxima over the keys each
// chunk block's rows see (the rescore flag's statistics).
//
// prefill_attn_kernel: one workgroup of 8 waves per (sequence, KV head, 32 query
// positions); wave w computes Q head 4*kv_head + (w & 3) for 16 positions.  The staged
// rows of each 64-key block are copied once per workgroup into LDS and used by all 4
// heads of the group and all 32 positions (gqa_kv_broadcast.v:38-59 at block scale).
// K runs one block ahead of V, so that each wave forms block j's probabilities while its
// MFMAs form block j+1's scores, then accumulates block j's V^T P^T.
//
//  * Scores S^T = K Q^T with v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims of K from
//    LDS (row = key), B = Q^T (column = query) held in registers.  Q is rotated and
//    scaled by scale*log2(e) in double, scaled by a power of two per query row, and split
//    into two fp16 parts (11-bit significands: ~22 bits of Q); the products are exact in
//    fp32.  Blocks with chunk keys add the trailing part of K against Q's leading part.
//    Lane (g, n) ends with the scores of keys 4g+i (i = 0..3) of each 16-key tile for
//    query n, times 2^(q scale + block K scale), which one multiply removes.
//  * Online softmax per query with an integer-valued running max (every rescale is an
//    exact power of two), p = exp2(s - m) in fp32, masked keys p = 0 exactly.
//  * O^T += V^T P^T with the same MFMA: A = 16 dims x 32 keys of V^T from LDS, B = P^T.
//    The lane already holds P for keys {4g+i} of tiles 2w and 2w+1, which is its B
//    operand for the 32-key window w if V^T stores each window's keys in that order
//    (slot 8g+4h+i <-> key 16h+4g+i).  P, scaled by 2^12, is split into two fp16 parts
//    (rounded to nearest: ~22 bits).  Each block's fp32 product is scaled by the block's
//    V scale into an fp64 accumulator, so accumulation over thousands of keys adds no fp32
//    rounding.
//  * O / l, rounded double -> f32 -> BF16, written in Q-head order; the row's rescore flag
//    decided from those BF16 values (pf_flag_row).
//
// Chunks of at most 16 new tokens take the multi-token decode path instead
// (gqa_multitoken.hip), which shares this file's LDS row layout (gqa_prefill_common.h).
#include "gqa_device.h"
#include "gqa_internal.h"
#include "gqa_prefill_common.h"

namespace gqa {

namespace {

constexpr int kPfPos = 32;                 // query positions per workgroup
constexpr int kPfWaves = 8;                // 4 Q heads x 2 tiles of 16 positions
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfBlk = 64;                 // keys per K/V block
constexpr int kStgThreads = 256;           // staging workgroup: 4 threads per row of a block
constexpr int kStgMaxWgs = 8192;
constexpr int kPScaleExp = 12;             // P is formed as 2^12 * 2^(s - m) <= 4096

size_t al256(size_t x) { return (x + 255) / 256 * 256; }

}  // namespace

// ---------------------------------------------------------------------------------
// Workspace of the prefill attention path: the rotated new K rows in fp32, the fp16 K and
// V planes, the trailing-part planes of the chunk blocks and the block scale words.
size_t prefill_stage_bytes(int32_t batch, int32_t n_new, int32_t capacity) {
    const size_t rows = static_cast<size_t>(batch) * n_new * kHkv;
    const size_t pos = (static_cast<size_t>(capacity) + kPfBlk - 1) / kPfBlk * kPfBlk;
    const size_t cb = static_cast<size_t>(prefill_chunk_blocks(n_new));
    const size_t bh = static_cast<size_t>(batch) * kHkv;
    return al256(rows * kD * sizeof(float)) + 2 * al256(bh * pos * kD * sizeof(uint16_t)) +
           al256(bh * cb * kPfBlk * kD * sizeof(uint16_t)) + al256(bh * (pos / kPfBlk) * sizeof(uint32_t));
}

void prefill_stage_layout(PrefillArgs& a, void* base) {
    const size_t rows = static_cast<size_t>(a.batch) * a.n_new * kHkv;
    a.stg_pos = (a.capacity + kPfBlk - 1) / kPfBlk * kPfBlk;
    a.stg_cb = prefill_chunk_blocks(a.n_new);
    const size_t bh = static_cast<size_t>(a.batch) * kHkv;
    char* p = static_cast<char*>(base);
    a.kx32 = reinterpret_cast<float*>(p);
    p += al256(rows * kD * sizeof(float));
    a.stg_k = reinterpret_cast<uint16_t*>(p);
    p += al256(bh * a.stg_pos * kD * sizeof(uint16_t));
    a.stg_v = reinterpret_cast<uint16_t*>(p);
    p += al256(bh * a.stg_pos * kD * sizeof(uint16_t));
    a.stg_klo = reinterpret_cast<uint16_t*>(p);
    p += al256(bh * a.stg_cb * kPfBlk * kD * sizeof(uint16_t));
    a.stg_scale = reinterpret_cast<uint32_t*>(p);
}

// ---------------------------------------------------------------------------------
// KV append: one wave per new (sequence, token); lane i computes the angle of frequency i
// at position start+t once (pyfiles/gen_gqa_wrapper_vectors.py:30-31) and rotates the
// pair (i, i+64) of all 8 KV heads' rows in double (:25-35).  All 8 heads' rows are
// requested before any is written, so a wave waits for memory once.
__global__ __launch_bounds__(256) void kv_append_kernel(PrefillArgs a) {
    const int64_t bt = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);   // b * T + t
    const int lane = threadIdx.x & (kWave - 1);
    if (blockIdx.x == 0) rs_clear(a, threadIdx.x);
    if (bt >= static_cast<int64_t>(a.batch) * a.n_new) return;
    const int t = static_cast<int>(bt % a.n_new);
    const int b = static_cast<int>(bt / a.n_new);
    // The rescore's counters start at zero (also for a sequence whose start is out of range:
    // the tile counters are indexed by tile, not by row).
    if (a.rs_hdr) {
        if (lane < kHq) a.rs_done[bt * kHq + lane] = 0u;
        if (t == 0 && lane < kHkv) a.rs_gcnt[b * kHkv + lane] = 0u;
    }
    const int st = a.start[b];
    if (!prefill_start_ok(a, st)) return;
    const int64_t pos = static_cast<int64_t>(st) + t;
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
    if (a.rs_hdr && any_rope) a.rs_cs[bt * kPairs + lane] = make_double2(cs, sn);
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
        if (ce[kvh] >= 0) {
            uint16_t* kdst = a.k + ce[kvh];
            uint16_t* vdst = a.v + ce[kvh];
            kdst[lane] = bf16_of(xr);
            kdst[lane + kPairs] = bf16_of(yr);
            vdst[lane] = vx[kvh];
            vdst[lane + kPairs] = vy[kvh];
        }
        if (a.kx32) {
            float* kr = a.kx32 + row * kD;
            kr[lane] = static_cast<float>(xr);
            kr[lane + kPairs] = static_cast<float>(yr);
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
// Staging.

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// Two floats -> two fp16 codes in one dword, each rounded to nearest (v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pk_f16(float lo, float hi) {
    f16x2_t h;
    h[0] = static_cast<_Float16>(lo);
    h[1] = static_cast<_Float16>(hi);
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ float f16_lo(uint32_t w) { return static_cast<float>(__builtin_bit_cast(f16x2_t, w)[0]); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return static_cast<float>(__builtin_bit_cast(f16x2_t, w)[1]); }

// x - (fp16 half of h), exact, in one instruction: v_fma_mix_f32 reads the half as fp16
// (op_sel_hi) and computes -h * 1 + x with one rounding, and x - h is representable.
__device__ __forceinline__ float sub_f16_lo(float x, uint32_t h) {
    float r;
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}
__device__ __forceinline__ float sub_f16_hi(float x, uint32_t h) {
    float r;
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
    return r;
}

// Scale exponent putting magnitude bits `mb` (fp32, sign cleared) in [2^14, 2^15): 14 - floor(log2).
// 0 for zero.  Exponents outside [-100, 100] mark the block (the attention kernel keeps the
// factor 2^-scale in the fp32 normal range) and are clamped.
__device__ __forceinline__ int stg_scale_exp(uint32_t mb, bool& bad) {
    if (mb == 0u) return 0;
    const int e = static_cast<int>(mb >> 23) - 127;
    if (e < -100 || e > 100) bad = true;
    return 14 - (e < -100 ? -100 : e > 100 ? 100 : e);
}

__device__ __forceinline__ float pow2f(int e) { return __uint_as_float(static_cast<uint32_t>(127 + e) << 23); }

// Statistics of one staged block for the rescore flag: thread (r, qq) holds pair groups 2qq
// and 2qq+1 of row r whole (dims 16qq .. 16qq+15 and 64+16qq ..), so its two squared group
// norms need no other thread, and the |V| codes of its 32 dims.  stg_stats_put writes the
// block's rows to LDS ([64 rows][64 dwords] of |V| codes, dword c = dims 2c and 2c+1; [64
// rows][8] norms) before the kernel's own barrier; after it, stg_stats_take reduces
// columns, one wave per 16 dword columns and 2 norm groups: a block of cached rows stores
// its maxima (rs_kblk / rs_dblk, folded over the cache by prefill_stat_reduce_kernel), a
// block holding chunk keys the maxima over its rows up to each row (rs_kpre / rs_dpre).
struct StgStatLds {
    uint32_t v[kPfBlk][kD / 2];
    uint32_t k[kPfBlk][8];
};

// n0, n1: the squared norms of pair groups 2qq and 2qq + 1 of the row's K; vw: its V as
// BF16 codes (dims 16qq .. +7, 16qq + 8 .., 64 + 16qq .., 64 + 16qq + 8 ..).
__device__ __forceinline__ void stg_stats_put(int r, int qq, float n0, float n1, const uint4 (&vw)[4],
                                              StgStatLds& sl) {
    uint4* vrow = reinterpret_cast<uint4*>(&sl.v[r][0]);
    const uint32_t m = 0x7fff7fffu;
    vrow[2 * qq] = make_uint4(vw[0].x & m, vw[0].y & m, vw[0].z & m, vw[0].w & m);
    vrow[2 * qq + 1] = make_uint4(vw[1].x & m, vw[1].y & m, vw[1].z & m, vw[1].w & m);
    vrow[8 + 2 * qq] = make_uint4(vw[2].x & m, vw[2].y & m, vw[2].z & m, vw[2].w & m);
    vrow[8 + 2 * qq + 1] = make_uint4(vw[3].x & m, vw[3].y & m, vw[3].z & m, vw[3].w & m);
    sl.k[r][2 * qq] = __float_as_uint(n0);
    sl.k[r][2 * qq + 1] = __float_as_uint(n1);
}

// Largest |x| over 8 BF16 codes, as fp32 bits (NaN and infinity above every finite value).
__device__ __forceinline__ uint32_t stg_absmax8(const uint4& w) {
    const uint32_t m = pk_max_u16(pk_max_u16(w.x & 0x7fff7fffu, w.y & 0x7fff7fffu),
                                  pk_max_u16(w.z & 0x7fff7fffu, w.w & 0x7fff7fffu));
    return max(m << 16, m & 0x7fff0000u);
}

// Two BF16 codes (one dword) times f, as two fp16 codes.
__device__ __forceinline__ uint32_t stg_f16x2(uint32_t w, float f) {
    return pk_f16(__uint_as_float(w << 16) * f, __uint_as_float(w & 0xffff0000u) * f);
}

__device__ __forceinline__ void stg_stats_take(const PrefillArgs& a, int bh, int blk, int st, int wave, int lane,
                                               const StgStatLds& sl) {
    // Wave w: |V| dword columns 16w .. 16w+15 (lane: column 16w + (lane & 15), rows
    // 16 (lane >> 4) .. +15) and norm groups 2w, 2w+1 (lane: group 2w + (lane & 1), rows
    // 2 (lane >> 1) and +1).
    const int col = 16 * wave + (lane & 15);
    const int rg = lane >> 4;
    const int kg = 2 * wave + (lane & 1);
    const int kr = 2 * (lane >> 1);
    if (blk * kPfBlk + kPfBlk - 1 < st) {
        uint32_t x = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) x = pk_max_u16(x, sl.v[16 * rg + i][col]);
        x = pk_max_u16(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), 16)));
        x = pk_max_u16(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), 32)));
        const int64_t e = static_cast<int64_t>(bh) * a.rs_nblk + blk;
        if (rg == 0) a.rs_dblk[e * (kD / 2) + col] = x;
        uint32_t y = max(sl.k[kr][kg], sl.k[kr + 1][kg]);
#pragma unroll
        for (int sh = 2; sh < kWave; sh <<= 1) y = max(y, static_cast<uint32_t>(__shfl_xor(static_cast<int>(y), sh)));
        if (lane < 2) a.rs_kblk[e * 8 + kg] = y;
        return;
    }
    // Running maxima down the rows: within each lane's 16 (or 2) rows, then the earlier
    // lanes' totals (row groups 16 and 32 lanes apart; norm rows 2, 4, .. lanes apart).
    const int cb = blk - st / kPfBlk;
    const int64_t e0 = (static_cast<int64_t>(bh) * a.rs_ncb + cb) * a.rs_nr;
    uint32_t run[16];
    uint32_t x = 0u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        x = pk_max_u16(x, sl.v[16 * rg + i][col]);
        run[i] = x;
    }
    uint32_t carry = 0u;
    {
        const uint32_t t16 = static_cast<uint32_t>(__shfl_up(static_cast<int>(x), 16));
        const uint32_t t32 = static_cast<uint32_t>(__shfl_up(static_cast<int>(x), 32));
        const uint32_t t48 = static_cast<uint32_t>(__shfl_up(static_cast<int>(x), 48));
        if (rg >= 1) carry = pk_max_u16(carry, t16);
        if (rg >= 2) carry = pk_max_u16(carry, t32);
        if (rg >= 3) carry = pk_max_u16(carry, t48);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
        *reinterpret_cast<uint32_t*>(a.rs_dpre + (e0 + 16 * rg + i) * kD + 2 * col) = pk_max_u16(run[i], carry);
    const uint32_t y0 = sl.k[kr][kg];
    const uint32_t y1 = max(y0, sl.k[kr + 1][kg]);
    uint32_t yc = 0u;
#pragma unroll
    for (int sh = 2; sh < kWave; sh <<= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(max(y1, yc)), sh));
        if (lane >= sh) yc = max(yc, o);
    }
    a.rs_kpre[(e0 + kr) * 8 + kg] = max(y0, yc);
    a.rs_kpre[(e0 + kr + 1) * 8 + kg] = max(y1, yc);
}

// One workgroup per (sequence, KV head, 64-position block) of the positions the attention
// reads, [0, start + T); thread (r, qq) holds dims 16qq .. 16qq+15 and 64+16qq .. of row r.
// Rows past start + T in the last block are written as zeros (the attention kernel copies
// whole blocks and masks them).
__global__ __launch_bounds__(kStgThreads) void prefill_stage_kernel(PrefillArgs a) {
    __shared__ uint32_t red[2][kStgThreads / kWave];
    __shared__ StgStatLds stat_s;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & (kWave - 1);
    const int r = tid >> 2;
    const int qq = tid & 3;
    const int nblk = a.stg_pos / kPfBlk;
    const int64_t n_items = static_cast<int64_t>(a.batch) * kHkv * nblk;
    for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int blk = static_cast<int>(item % nblk);
        const int bh = static_cast<int>(item / nblk);
        const int b = bh / kHkv;
        const int h = bh % kHkv;
        const int st = a.start[b];
        if (!prefill_start_ok(a, st)) continue;
        const int n_keys = st + a.n_new;
        if (blk * kPfBlk >= n_keys) continue;
        const int p = blk * kPfBlk + r;
        // This thread's 32 dims of the row (16-byte pieces c: dims 16qq + 8c for c < 2, 64 +
        // 16qq + 8(c - 2) after): V and cached K kept as BF16 codes; a chunk row's K (fp32,
        // from the append) is read here for its maxima and norms and again for conversion.
        uint4 vw[4], kw[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) vw[c] = kw[c] = make_uint4(0u, 0u, 0u, 0u);
        bool bad = false;
        const bool chunk_row = p >= st && p < n_keys;
        const float* kx = a.kx32 + ((static_cast<int64_t>(b) * a.n_new + (p - st)) * kHkv + h) * kD;
        uint32_t rk = 0u, rv = 0u;
        float n0 = 0.f, n1 = 0.f;
        if (p < n_keys) {
            const int64_t ce = cache_elem(a, b, h, p);
            if (ce < 0) {
                bad = true;
            } else {
                const char* vr = reinterpret_cast<const char*>(a.v + ce);
#pragma unroll
                for (int c = 0; c < 4; ++c) vw[c] = load_stream16(vr + 128 * (c >> 1) + 32 * qq + 16 * (c & 1));
                if (!chunk_row) {
                    const char* kr = reinterpret_cast<const char*>(a.k + ce);
#pragma unroll
                    for (int c = 0; c < 4; ++c) kw[c] = load_stream16(kr + 128 * (c >> 1) + 32 * qq + 16 * (c & 1));
                    rk = max(max(stg_absmax8(kw[0]), stg_absmax8(kw[1])), max(stg_absmax8(kw[2]), stg_absmax8(kw[3])));
                    const uint32_t g0[8] = {kw[0].x, kw[0].y, kw[0].z, kw[0].w, kw[2].x, kw[2].y, kw[2].z, kw[2].w};
                    const uint32_t g1[8] = {kw[1].x, kw[1].y, kw[1].z, kw[1].w, kw[3].x, kw[3].y, kw[3].z, kw[3].w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        n0 = bf16x2_sq_acc(g0[i], n0);
                        n1 = bf16x2_sq_acc(g1[i], n1);
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        // dims 16qq + 4c (c < 4), 64 + 16qq + 4(c - 4): groups 2qq + ((c >> 1) & 1)
                        const float4 f = *reinterpret_cast<const float4*>(kx + 64 * (c >> 2) + 16 * qq + 4 * (c & 3));
                        rk = max(rk, max(max(__float_as_uint(f.x) & 0x7fffffffu, __float_as_uint(f.y) & 0x7fffffffu),
                                         max(__float_as_uint(f.z) & 0x7fffffffu, __float_as_uint(f.w) & 0x7fffffffu)));
                        const float sq = fmaf(f.x, f.x, fmaf(f.y, f.y, fmaf(f.z, f.z, f.w * f.w)));
                        if ((c >> 1) & 1) n1 += sq;
                        else n0 += sq;
                    }
                }
                rv = max(max(stg_absmax8(vw[0]), stg_absmax8(vw[1])), max(stg_absmax8(vw[2]), stg_absmax8(vw[3])));
            }
        }
        // Largest magnitudes as fp32 bit patterns: per row over its four threads, then over
        // the block.
        rk = max(rk, static_cast<uint32_t>(__shfl_xor(static_cast<int>(rk), 1)));
        rk = max(rk, static_cast<uint32_t>(__shfl_xor(static_cast<int>(rk), 2)));
        rv = max(rv, static_cast<uint32_t>(__shfl_xor(static_cast<int>(rv), 1)));
        rv = max(rv, static_cast<uint32_t>(__shfl_xor(static_cast<int>(rv), 2)));
        uint32_t wk = rk, wv = rv;
#pragma unroll
        for (int sh = 4; sh < kWave; sh <<= 1) {
            wk = max(wk, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wk), sh)));
            wv = max(wv, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wv), sh)));
        }
        __syncthreads();                      // red and stat_s are rewritten for every item
        if (lane == 0) {
            red[0][wave] = wk;
            red[1][wave] = wv;
        }
        if (a.rs_hdr) stg_stats_put(r, qq, n0, n1, vw, stat_s);
        __syncthreads();
        uint32_t bk = 0u, bv = 0u;
#pragma unroll
        for (int w = 0; w < kStgThreads / kWave; ++w) {
            bk = max(bk, red[0][w]);
            bv = max(bv, red[1][w]);
        }
        if (bk >= 0x7f800000u || bv >= 0x7f800000u) bad = true;
        const int sk = stg_scale_exp(bk, bad);
        const int sv = stg_scale_exp(bv, bad);
        // A row far below the block's largest magnitude would keep fewer bits of its small
        // elements than the attention's error bound allows.
        if (bk >= (13u << 23) && rk != 0u && rk < bk - (12u << 23)) bad = true;
        if (bv >= (13u << 23) && rv != 0u && rv < bv - (12u << 23)) bad = true;
        const bool any_bad = __syncthreads_or(bad);
        const float fk = pow2f(sk), fv = pow2f(sv);
        const int64_t row = static_cast<int64_t>(bh) * a.stg_pos + p;
        char* ko = reinterpret_cast<char*>(a.stg_k + row * kD);
        char* vo = reinterpret_cast<char*>(a.stg_v + row * kD);
        const bool chunk_blk = blk * kPfBlk + kPfBlk - 1 >= st;
        char* lo = reinterpret_cast<char*>(
            a.stg_klo + ((static_cast<int64_t>(bh) * a.stg_cb + (blk - st / kPfBlk)) * kPfBlk + r) * kD);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int off = 128 * (c >> 1) + 32 * qq + 16 * (c & 1);
            *reinterpret_cast<uint4*>(vo + off) = make_uint4(stg_f16x2(vw[c].x, fv), stg_f16x2(vw[c].y, fv),
                                                             stg_f16x2(vw[c].z, fv), stg_f16x2(vw[c].w, fv));
            uint4 kh, kl = make_uint4(0u, 0u, 0u, 0u);
            if (!chunk_row) {
                kh = make_uint4(stg_f16x2(kw[c].x, fk), stg_f16x2(kw[c].y, fk), stg_f16x2(kw[c].z, fk),
                                stg_f16x2(kw[c].w, fk));
            } else {
                // the fp32 row as two fp16 parts (leading, trailing)
                const float* src = kx + 64 * (c >> 1) + 16 * qq + 8 * (c & 1);
                const float4 f0 = *reinterpret_cast<const float4*>(src);
                const float4 f1 = *reinterpret_cast<const float4*>(src + 4);
                const float x[8] = {f0.x * fk, f0.y * fk, f0.z * fk, f0.w * fk, f1.x * fk, f1.y * fk, f1.z * fk, f1.w * fk};
                uint32_t hh[4], ll[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    hh[j] = pk_f16(x[2 * j], x[2 * j + 1]);
                    ll[j] = pk_f16(x[2 * j] - f16_lo(hh[j]), x[2 * j + 1] - f16_hi(hh[j]));
                }
                kh = make_uint4(hh[0], hh[1], hh[2], hh[3]);
                kl = make_uint4(ll[0], ll[1], ll[2], ll[3]);
            }
            *reinterpret_cast<uint4*>(ko + off) = kh;
            if (chunk_blk) *reinterpret_cast<uint4*>(lo + off) = kl;
        }
        if (tid == 0)
            a.stg_scale[static_cast<int64_t>(bh) * nblk + blk] =
                (static_cast<uint32_t>(sk) & 0xffu) | ((static_cast<uint32_t>(sv) & 0xffu) << 8) |
                (any_bad ? 0x80000000u : 0u);
        if (a.rs_hdr) stg_stats_take(a, bh, blk, st, wave, lane, stat_s);
    }
}

// The maxima over the keys before each chunk block of a (sequence, KV head): the blocks of
// cached rows only (the block maxima the staging kernel wrote) folded by 16 partial sweeps
// (thread t: dword column t % 64 of every 16th block; norm group t % 8 of every 64th),
// meeting in LDS; then, chunk block by chunk block, the previous chunk blocks' maxima (row
// 63 of their running maxima).
__global__ __launch_bounds__(1024) void prefill_stat_reduce_kernel(PrefillArgs a) {
    __shared__ uint32_t vpart[16][kD / 2];
    __shared__ uint32_t kpart[64][8];
    const int bh = blockIdx.x;
    const int tid = threadIdx.x;
    const int st = a.start[bh / kHkv];
    const int n_cached = prefill_start_ok(a, st) ? st / kPfBlk : 0;
    {
        const int col = tid & 63, sub = tid >> 6;
        const uint32_t* vb = a.rs_dblk + static_cast<int64_t>(bh) * a.rs_nblk * (kD / 2) + col;
        uint32_t x = 0u;
        for (int i0 = sub; i0 < n_cached; i0 += 16 * 8) {
            uint32_t w[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                w[j] = i0 + 16 * j < n_cached ? vb[static_cast<int64_t>(i0 + 16 * j) * (kD / 2)] : 0u;
#pragma unroll
            for (int j = 0; j < 8; ++j) x = pk_max_u16(x, w[j]);
        }
        vpart[sub][col] = x;
    }
    if (tid < 512) {
        const int g = tid & 7, ks = tid >> 3;
        const uint32_t* kb = a.rs_kblk + static_cast<int64_t>(bh) * a.rs_nblk * 8 + g;
        uint32_t y = 0u;
        for (int i0 = ks; i0 < n_cached; i0 += 64 * 4) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = i0 + 64 * j < n_cached ? kb[static_cast<int64_t>(i0 + 64 * j) * 8] : 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) y = max(y, w[j]);
        }
        kpart[ks][g] = y;
    }
    __syncthreads();
    if (tid < kD / 2) {
        uint32_t v = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) v = pk_max_u16(v, vpart[i][tid]);
        // Chunk block cb: the cached maxima and chunk blocks 0 .. cb-1 (their last row).
        const int64_t pre0 = static_cast<int64_t>(bh) * a.rs_ncb * a.rs_nr;
        for (int cb = 0; cb < a.rs_ncb; ++cb) {
            uint32_t* dc = a.rs_dc + (static_cast<int64_t>(bh) * a.rs_ncb + cb) * kD + 2 * tid;
            dc[0] = v & 0xffffu;
            dc[1] = v >> 16;
            v = pk_max_u16(v, *reinterpret_cast<const uint32_t*>(a.rs_dpre + (pre0 + static_cast<int64_t>(cb) * a.rs_nr + a.rs_nr - 1) * kD + 2 * tid));
        }
    } else if (tid < kD / 2 + 8) {
        const int g = tid - kD / 2;
        uint32_t y = 0u;
#pragma unroll 8
        for (int i = 0; i < 64; ++i) y = max(y, kpart[i][g]);
        const int64_t pre0 = static_cast<int64_t>(bh) * a.rs_ncb * a.rs_nr;
        for (int cb = 0; cb < a.rs_ncb; ++cb) {
            a.rs_kc[(static_cast<int64_t>(bh) * a.rs_ncb + cb) * 8 + g] = y;
            y = max(y, a.rs_kpre[(pre0 + static_cast<int64_t>(cb) * a.rs_nr + a.rs_nr - 1) * 8 + g]);
        }
    }
}

hipError_t launch_prefill_stat_reduce(const PrefillArgs& a, hipStream_t stream) {
    if (!a.rs_hdr) return hipSuccess;
    hipLaunchKernelGGL(prefill_stat_reduce_kernel, dim3(static_cast<unsigned>(a.batch * kHkv)), dim3(1024), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_prefill_stage(const PrefillArgs& a, hipStream_t stream) {
    const int64_t n_items = static_cast<int64_t>(a.batch) * kHkv * (a.stg_pos / kPfBlk);
    if (n_items == 0) return hipSuccess;
    const int64_t grid = n_items < kStgMaxWgs ? n_items : kStgMaxWgs;
    hipLaunchKernelGGL(prefill_stage_kernel, dim3(static_cast<unsigned>(grid)), dim3(kStgThreads), 0, stream, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Attention.

// LDS: six 16 KB planes of 64 rows x 256 B -- K of buffers 0 and 1, V of buffers 0 and 1,
// the trailing parts of chunk keys for buffers 0 and 1 (96 KB in all).  K runs one block
// ahead of V: while block j's probabilities are formed and its V^T P^T accumulated, block
// j+1's scores are formed from the other K buffer.  Rows are copied from the staging planes
// straight into LDS (global_load_lds_dwordx4: lane l of an instruction writes bytes
// [16l, 16l + 16) of a 1 KB stretch = 4 rows), so a row's 16 16-byte chunks are placed by
// choosing which chunk each lane fetches: chunk c of row r sits at position c ^ pf_swz(r & 15).
// With that swizzle the K operand reads (16 rows, one chunk) and the V^T transpose reads
// (16 rows, two chunks) hit 64 distinct banks per pass, and because it depends on r & 15 only,
// the rows 16 apart that one lane reads differ by a constant offset.
constexpr int kPlaneB = kPfBlk * kRowB;     // 16 KB per plane
constexpr int kOffK = 0;                    // + buffer * kPlaneB
constexpr int kOffV = 2 * kPlaneB;
constexpr int kOffKlo = 4 * kPlaneB;
// Then a ring of block scale words: words for blocks [0, 512) are copied at the start and
// words for blocks [256k + 256, 256k + 512) at step 256k, into the half whose blocks are done,
// so that a word is in LDS 255 steps before it is read.  Copied like the rows (straight into
// LDS, completed by the step's vmcnt(0) wait), it costs no wait of its own: a plain load's
// wait would also wait for the K/V copies in flight.
constexpr int kOffSw = 6 * kPlaneB;
constexpr int kSwRing = 512;
constexpr int kLdsB = 6 * kPlaneB + kSwRing * 4;

// Wave w of the workgroup copies rows 8w .. 8w+7 of a plane (two 4-row instructions).
__device__ __forceinline__ int pf_copy_row(int wave, int ii, int lane) { return 4 * (2 * wave + ii) + (lane >> 4); }

// The lane's byte offset within a staged 64-row block for its two copy instructions.
__device__ __forceinline__ void pf_copy_offsets(int wave, int lane, uint32_t (&loff)[2]) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int r = pf_copy_row(wave, ii, lane);
        loff[ii] = static_cast<uint32_t>(r * kRowB + 16 * ((lane & 15) ^ pf_swz(r)));
    }
}

// Request one staged 64-row block (16 KB at `src`) into the LDS plane at `dst`.
__device__ __forceinline__ void pf_issue(const char* src, const uint32_t (&loff)[2], uint8_t* dst, int wave) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
        __builtin_amdgcn_global_load_lds(src + loff[ii], (lds_void_t*)(dst + (2 * wave + ii) * 1024), 16, 0, 0);
}

__device__ __forceinline__ f16x8_t as_f16x8(const uint4& w) { return __builtin_bit_cast(f16x8_t, w); }

// 8 fp16 K values of row `row`, bytes [16 chunk, 16 chunk + 16) of the plane at `plane`.
__device__ __forceinline__ f16x8_t pf_k16(const uint8_t* plane, int row, int chunk) {
    return *reinterpret_cast<const f16x8_t*>(plane + row * kRowB + 16 * (chunk ^ pf_swz(row)));
}

// One 32-dim slice (dims 32q .. 32q+31) of the scores S^T[key][query] of one 16-query tile
// over the block's 4 key tiles: the 2 fp16 parts of Q against the K plane, and for chunk
// keys the trailing part of K against Q's leading part.
template <bool kNew>
__device__ __forceinline__ void pf_qk_slice(const uint8_t* kplane, const f16x8_t (&qop)[2][4], int q, int n,
                                            int g, f32x4_t (&sacc)[4]) {
    f16x8_t ak[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k16(kplane, 16 * kt + n, 4 * q + g);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
            sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak[kt], qop[s][q], sacc[kt], 0, 0, 0);
    if (kNew) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k16(kplane + (kOffKlo - kOffK), 16 * kt + n, 4 * q + g);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
            sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak[kt], qop[0][q], sacc[kt], 0, 0, 0);
    }
}

// Per-tile softmax state: the running max (integer-valued, log2 units), sum and O (fp64,
// lane (g, n): O^T[16dt + 4g + i][query n]), both in units of 2^12 p, and the fp32 sum of
// V^T P^T over the current group of up to kPfGroup blocks (moved into the fp64 O when the
// group closes: fp32 sums over 256 keys add no error measurable against per-block sums).
constexpr int kPfGroup = 4;
struct PfTile {
    double o64[8][4];
    f32x4_t acc[8];
    double l64;
    float m_run;
    float u;           // bound on what fp16's subnormal quantum adds to O (O's units, this lane's keys)
};

// Closes a group: O += acc * cv (cv = 2^-(V scale of the group's blocks), exact).
__device__ __forceinline__ void pf_flush(PfTile& t, double cv) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) t.o64[dt][i] = fma(static_cast<double>(t.acc[dt][i]), cv, t.o64[dt][i]);
        t.acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
}

// Running max after a block: masks keys past each query on diagonal blocks, then returns
// ceil(block max) where that exceeds the running max m (integer-valued, so every rescale is an
// exact power of two), else m.  `mult` turns the block's raw scores into log2 units.  The two
// cross-row steps are gfx950 lane swaps (rows 16 and 32 lanes apart), not LDS permutes.
__device__ __forceinline__ float pf_next_max(f32x4_t (&sacc)[4], bool diag, int key0, int g, int pos_n, float m,
                                             float mult) {
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
    bmax = fmaxf(__uint_as_float(x32[0]), __uint_as_float(x32[1])) * mult;
    return bmax > m ? ceilf(bmax) : m;
}

// Moves O, the open group's sum and l to the running max m_new (exact power-of-two scaling;
// an fp32 group term pushed below 2^-149 is below 2^-149 of the new maximum's weight).
__device__ __forceinline__ void pf_rescale(PfTile& t, float m_new) {
    if (__ballot(m_new != t.m_run)) {
        const int shift = (t.m_run == -INFINITY) ? 0 : max_shift(t.m_run, m_new);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                t.o64[dt][i] = ldexp(t.o64[dt][i], shift);
                t.acc[dt][i] = ldexpf(t.acc[dt][i], shift);
            }
        t.l64 = ldexp(t.l64, shift);
        t.u = ldexpf(t.u, shift);
        t.m_run = m_new;
    }
}

// p = 2^12 * 2^(s - m) of key tile kt (0 for masked keys; s = raw score * mult), summed into
// lsum and split into two fp16 parts rounded to nearest (p = p1 + p2 to 2^-22 relative),
// packed as the P^T B operand: ph[part][window][dword].
__device__ __forceinline__ void pf_probs_tile16(const f32x4_t& s, float mult, float off, float& lsum,
                                                uint32_t (&ph)[2][2][4], int kt) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // v_exp_f32: 2^x, 0 for -inf (masked keys); results below 2^-126 flush to 0.
        p[i] = __builtin_amdgcn_exp2f(fmaf(s[i], mult, off));
        lsum += p[i];
    }
    const int w = kt >> 1, d0 = (kt & 1) * 2;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t h1 = pk_f16(p[2 * j], p[2 * j + 1]);
        ph[0][w][d0 + j] = h1;
        ph[1][w][d0 + j] = pk_f16(sub_f16_lo(p[2 * j], h1), sub_f16_hi(p[2 * j + 1], h1));
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

__device__ __forceinline__ f16x8_t pf_vt_operand(const VtPair& v, int w) {
    union {
        short4_t h[2];
        f16x8_t v;
    } u;
    u.h[0] = v.r[w][0];
    u.h[1] = v.r[w][1];
    return u.v;
}

// Per-lane LDS address of the transpose reads of dim tile dt (V buffer 0, window 0).
__device__ __forceinline__ uint32_t pf_vt_addr(uint32_t lds_base, int dt, int lane) {
    return lds_base + kOffV + vt_tr_offset(dt, lane);
}

// The group's fp32 sum += the block's V^T P^T: per 16-dim tile, V^T (transpose reads) against
// the two P parts of both 32-key windows; two tiles at a time, the next two tiles' operands
// requested before the current two's products.
__device__ __forceinline__ void pf_pv(const uint32_t (&vaddr)[8], uint32_t voff, const uint32_t (&ph)[2][2][4],
                                      PfTile& t) {
    f16x8_t pb[2][2];
#pragma unroll
    for (int w = 0; w < 2; ++w)
#pragma unroll
        for (int s = 0; s < 2; ++s) pb[w][s] = as_f16x8(make_uint4(ph[s][w][0], ph[s][w][1], ph[s][w][2], ph[s][w][3]));
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
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    t.acc[d0 + e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf_vt_operand(cur[e], w), pb[w][s],
                                                                           t.acc[d0 + e], 0, 0, 0);
        if (d0 + 2 < 8) {
            cur[0] = nxt[0];
            cur[1] = nxt[1];
        }
    }
}

// Probabilities of the current block (raw scores `scur` times `mult`, running max already
// grown) interleaved with the scores of the next block from K buffer `kplane` (kNext: there
// is one; kNew: it holds chunk keys).
template <bool kNext, bool kNew>
__device__ __forceinline__ void pf_probs_and_next(const f32x4_t (&scur)[4], float mult, float vshift,
                                                  const uint8_t* kplane, const f16x8_t (&qop)[2][4], int n, int g,
                                                  PfTile& t, uint32_t (&ph)[2][2][4], f32x4_t (&snext)[4]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) snext[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
    // p carries 2^vshift more (the group's V scale over this block's, |vshift| <= 3); l does not
    const float off = static_cast<float>(kPScaleExp) - t.m_run + vshift;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (kNext) pf_qk_slice<kNew>(kplane, qop, q, n, g, snext);
        pf_probs_tile16(scur[q], mult, off, lsum, ph, q);
    }
    t.l64 += ldexp(static_cast<double>(lsum), -static_cast<int>(vshift));
}

// The rescore flag of one output row, in the attention kernel's layout: lane (g, n) holds
// dims 16 dt + 4 g + i of query n's row (BF16 codes, pk[dt]).  The same decision as the
// multi-token merge's (rs_flag_decide over the row's elements in units of each dim's largest |V|
// and the scores' bound E = scale log2(e) sum_G |q_G| max|k_G|), over the keys the row at
// position pos sees: the keys before its chunk block (rs_kc, rs_dc at that block, reduced
// before this kernel runs) and the block's rows up to its own (rs_kpre, rs_dpre).  Q's
// pair-group norms come from the row as given (rotation leaves them unchanged): this lane
// reads dims 8g .. 8g+7 and 32 + 8g .. (and their pairs 64 on), pair groups g and 4 + g.
// y and its square in double, as in the multi-token merge (in fp32 y^2 underflows in every
// dim of a row whose elements lie ~2^63 below their dims' largest |V|).  ul bounds the error
// fp16's subnormal quantum added to every element (the attention loop's u over l): a row
// with an element below 8 ul, where that error could reach 64 ULP with a margin of 2, is
// rescored as well.  Returns the decision for the row in every lane of its column.
__device__ __forceinline__ bool pf_flag_row(const PrefillArgs& a, int b, int kvh, int st, int pos, int64_t row,
                                            float m, bool forced, double ul, const uint2 (&pk)[8], int lane) {
    const int g = lane >> 4;
    const int cb = pos / kPfBlk - st / kPfBlk;
    const int r = pos % kPfBlk;
    const int64_t ec = (static_cast<int64_t>(b) * kHkv + kvh) * a.rs_ncb + cb;
    const int64_t er = ec * a.rs_nr + r;
    const uint16_t* qrow = a.q + row * kD;
    const uint4 q0 = *reinterpret_cast<const uint4*>(qrow + 8 * g);
    const uint4 q1 = *reinterpret_cast<const uint4*>(qrow + 32 + 8 * g);
    const uint4 q2 = *reinterpret_cast<const uint4*>(qrow + kPairs + 8 * g);
    const uint4 q3 = *reinterpret_cast<const uint4*>(qrow + kPairs + 32 + 8 * g);
    const uint32_t k0 = max(a.rs_kc[ec * 8 + g], a.rs_kpre[er * 8 + g]);
    const uint32_t k1 = max(a.rs_kc[ec * 8 + 4 + g], a.rs_kpre[er * 8 + 4 + g]);
    double ss = 0.0, mn2 = INFINITY;
    float mnx = INFINITY;
    bool bad = forced, vinf = false;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
        const uint4 dc = *reinterpret_cast<const uint4*>(a.rs_dc + ec * kD + 16 * dt + 4 * g);
        const uint2 dp = *reinterpret_cast<const uint2*>(a.rs_dpre + er * kD + 16 * dt + 4 * g);
        const uint32_t d[4] = {max(dc.x, dp.x & 0xffffu), max(dc.y, dp.x >> 16), max(dc.z, dp.y & 0xffffu),
                               max(dc.w, dp.y >> 16)};
        const uint32_t xs[4] = {pk[dt].x << 16, pk[dt].x & 0xffff0000u, pk[dt].y << 16, pk[dt].y & 0xffff0000u};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = __uint_as_float(xs[i]);
            const float dv = __uint_as_float(d[i] << 16);
            const double y = dv > 0.f ? static_cast<double>(x) * __builtin_amdgcn_rcp(static_cast<double>(dv)) : 0.0;
            ss = fma(y, y, ss);
            if (dv > 0.f) mn2 = fmin(mn2, y * y);
            mnx = fminf(mnx, fabsf(x));
            bad |= !__builtin_isfinite(x);
            vinf |= !(dv <= 3.4028235e38f);         // an infinite or NaN V among the row's keys
        }
    }
    float qq0 = 0.f, qq1 = 0.f;
    {
        const uint32_t w0[8] = {q0.x, q0.y, q0.z, q0.w, q2.x, q2.y, q2.z, q2.w};
        const uint32_t w1[8] = {q1.x, q1.y, q1.z, q1.w, q3.x, q3.y, q3.z, q3.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            qq0 = bf16x2_sq_acc(w0[i], qq0);
            qq1 = bf16x2_sq_acc(w1[i], qq1);
        }
    }
    float e = sqrtf(qq0) * sqrtf(__uint_as_float(k0)) + sqrtf(qq1) * sqrtf(__uint_as_float(k1));
    // the row's four lanes: n, n + 16, n + 32, n + 48
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    e += __shfl_xor(e, 16);
    e += __shfl_xor(e, 32);
    mn2 = fmin(mn2, __shfl_xor(mn2, 16));
    mn2 = fmin(mn2, __shfl_xor(mn2, 32));
    mnx = fminf(mnx, __shfl_xor(mnx, 16));
    mnx = fminf(mnx, __shfl_xor(mnx, 32));
    bad |= static_cast<double>(mnx) < 8.0 * ul;
    bad = (__shfl_xor(static_cast<int>(bad), 16) | __shfl_xor(static_cast<int>(bad), 32) |
           __shfl_xor(static_cast<int>(bad), 48) | static_cast<int>(bad)) != 0;
    vinf = (__shfl_xor(static_cast<int>(vinf), 16) | __shfl_xor(static_cast<int>(vinf), 32) |
            __shfl_xor(static_cast<int>(vinf), 48) | static_cast<int>(vinf)) != 0;
    if (vinf && (lane >> 4) == 0) atomicOr(a.rs_hdr + 2, 1u);   // the row is flagged: y = 0 there
    return bad || rs_flag_decide(mn2, ss, static_cast<double>(m), static_cast<double>(e) * fabs(a.qk_scale_log2));
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
    const int nblk_stg = a.stg_pos / kPfBlk;
    const char* kseg = reinterpret_cast<const char*>(a.stg_k + static_cast<int64_t>(pair) * a.stg_pos * kD);
    const char* vseg = reinterpret_cast<const char*>(a.stg_v + static_cast<int64_t>(pair) * a.stg_pos * kD);
    const char* kloseg = reinterpret_cast<const char*>(a.stg_klo + static_cast<int64_t>(pair) * a.stg_cb * kPfBlk * kD);
    const uint32_t* sw = a.stg_scale + static_cast<int64_t>(pair) * nblk_stg;
    const int cb0 = st / kPfBlk;            // first block holding chunk keys
    auto blk_new = [&](int blk) { return blk >= cb0; };
    auto blk_diag = [&](int blk) { return blk * kPfBlk + kPfBlk - 1 > st + t_wave0; };
    auto issue_k = [&](int blk, int buf, const uint32_t (&loff)[2]) {
        pf_issue(kseg + static_cast<int64_t>(blk) * kPlaneB, loff, lds + kOffK + buf * kPlaneB, wave);
        if (blk_new(blk))
            pf_issue(kloseg + static_cast<int64_t>(blk - cb0) * kPlaneB, loff, lds + kOffKlo + buf * kPlaneB, wave);
    };
    auto issue_v = [&](int blk, int buf, const uint32_t (&loff)[2]) {
        pf_issue(vseg + static_cast<int64_t>(blk) * kPlaneB, loff, lds + kOffV + buf * kPlaneB, wave);
    };

    // K of blocks 0 and 1 and V of block 0 are requested before the Q operands are formed.
    uint32_t loff[2];
    pf_copy_offsets(wave, lane, loff);
    issue_k(0, 0, loff);
    issue_v(0, 0, loff);
    if (n_blk > 1) issue_k(1, 1, loff);
    // Scale words of blocks 64 wave .. 64 wave + 63 (entries past the last block repeat it).
    auto issue_sw = [&](int first) {
        __builtin_amdgcn_global_load_lds(sw + min(first + lane, nblk_stg - 1),
                                         (lds_void_t*)(lds + kOffSw + 4 * (first & (kSwRing - 1))), 4, 0, 0);
    };
    issue_sw(64 * wave);
    auto sw_at = [&](int blk) {
        return __builtin_amdgcn_readfirstlane(
            *reinterpret_cast<const uint32_t*>(lds + kOffSw + 4 * (blk & (kSwRing - 1))));
    };

    // Q operands: query n = this lane's column, dims 32kb + 8g + j, two fp16 parts of Q
    // scaled by 2^sq, sq putting the row's largest magnitude in [2^14, 2^15).
    f16x8_t qop[2][4];
    float cq;                               // 2^-sq
    bool q_bad = false;
    {
        const uint16_t* qrow = a.q + ((static_cast<int64_t>(b) * T + tq_c) * kHq + hq) * kD;
        // Every load first (the rotation below branches inside sincos, and each branch would
        // otherwise wait for all memory in flight, the K/V copies included).
        uint16_t qx[2][8], qy[2][8];
        double fr[2][8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = 32 * kb + 8 * g + j;
                qx[kb][j] = qrow[d];
                qy[kb][j] = qrow[d + kPairs];
                fr[kb][j] = a.rope.inv_freq[d];
            }
        double qv[4][8];
        double mx = 0.0;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const double x = bf16_to_f32(qx[kb][j]);
                const double y = bf16_to_f32(qy[kb][j]);
                double xr = x, yr = y;
                if (a.flags & 1u) rope_pair(x, y, pos_n, fr[kb][j], xr, yr);
                qv[kb][j] = xr * a.qk_scale_log2;
                qv[kb + 2][j] = yr * a.qk_scale_log2;
                // NaN fails both comparisons
                if (!(fabs(qv[kb][j]) <= 1e300) || !(fabs(qv[kb + 2][j]) <= 1e300)) q_bad = true;
                mx = fmax(mx, fmax(fabs(qv[kb][j]), fabs(qv[kb + 2][j])));
            }
        }
        mx = fmax(mx, __shfl_xor(mx, 16));
        mx = fmax(mx, __shfl_xor(mx, 32));
        int e = 0;
        if (mx > 0.0) {
            e = ilogb(mx);
            if (e < -100 || e > 100) q_bad = true;
            e = e < -100 ? -100 : e > 100 ? 100 : e;
        }
        const int sq = mx > 0.0 ? 14 - e : 0;
        cq = pow2f(-sq);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            uint32_t w0[4], w1[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const double x0 = ldexp(qv[kb][2 * j], sq), x1 = ldexp(qv[kb][2 * j + 1], sq);
                const _Float16 h0 = static_cast<_Float16>(static_cast<float>(x0));
                const _Float16 h1 = static_cast<_Float16>(static_cast<float>(x1));
                f16x2_t hh;
                hh[0] = h0;
                hh[1] = h1;
                w0[j] = __builtin_bit_cast(uint32_t, hh);
                w1[j] = pk_f16(static_cast<float>(x0 - static_cast<double>(h0)),
                               static_cast<float>(x1 - static_cast<double>(h1)));
            }
            // Pin the operands: without this the compiler re-derives them from the double
            // rows inside the block loop to save registers.
            asm volatile("" : "+v"(w0[0]), "+v"(w0[1]), "+v"(w0[2]), "+v"(w0[3]));
            asm volatile("" : "+v"(w1[0]), "+v"(w1[1]), "+v"(w1[2]), "+v"(w1[3]));
            qop[0][kb] = as_f16x8(make_uint4(w0[0], w0[1], w0[2], w0[3]));
            qop[1][kb] = as_f16x8(make_uint4(w1[0], w1[1], w1[2], w1[3]));
        }
    }

    const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(lds)));
    uint32_t vaddr[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) vaddr[dt] = pf_vt_addr(lds_base, dt, lane);

    PfTile tl;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) tl.o64[dt][i] = 0.0;
        tl.acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    tl.l64 = 0.0;
    tl.m_run = -INFINITY;
    tl.u = 0.f;
    // The open group: blocks summed into tl.acc so far and their V scale exponent.  A block
    // whose V scale differs from the group's by more than 3 (its P would leave fp16's range
    // or its precision) closes the group first.  A block holding chunk keys is summed alone:
    // its scales depend on rows that later tokens see and this token does not, and within a
    // group a different scale would change how the other blocks' terms round, so this
    // token's output would depend on keys its mask hides.  Alone, its sum only scales by a
    // power of two.
    int grp_n = 0, grp_sv = 0;

    // Raw scores carry 2^(sq + sk): mult = 2^-sq * 2^-sk(block) turns them into log2 units.
    // (Kept at least 2^-126: a smaller factor means scores below ~2^-90, all p = 1 either way,
    // and 0 would turn masked keys' -inf into NaN.)
    auto blk_mult = [&](uint32_t w) {
        return fmaxf(cq * pow2f(-static_cast<int>(static_cast<int8_t>(w & 0xffu))), 1.17549435e-38f);
    };
    auto blk_sv = [&](uint32_t w) { return static_cast<int>(static_cast<int8_t>((w >> 8) & 0xffu)); };
    // The largest V scale exponent among this workgroup's blocks (the smallest-V block's).
    int sv_hi = -128;
    for (int j = lane; j < n_blk; j += kWave) sv_hi = max(sv_hi, blk_sv(sw[j]));
#pragma unroll
    for (int sh = 1; sh < kWave; sh <<= 1) sv_hi = max(sv_hi, __shfl_xor(sv_hi, sh));
    sv_hi = __builtin_amdgcn_readfirstlane(sv_hi);

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
    uint32_t w_cur = sw_at(0);
    uint32_t unsafe = w_cur;                // bit 31 of any block read marks all rows
    float mult_cur = blk_mult(w_cur);
    pf_rescale(tl, pf_next_max(scur, blk_diag(0), 0, g, pos_n, tl.m_run, mult_cur));
    __syncthreads();

    for (int blk = 0; blk < n_blk; ++blk) {
        // Resident: K of block blk+1 (K buffer (blk+1)&1) and V of block blk (V buffer blk&1).
        // Free: K buffer blk&1 (block blk, scored in the previous step) and V buffer
        // (blk+1)&1 (block blk-1).
        if (blk + 2 < n_blk) issue_k(blk + 2, blk & 1, loff);
        if (blk + 1 < n_blk) issue_v(blk + 1, (blk + 1) & 1, loff);
        if ((blk & 255) == 0 && blk > 0 && wave < 4 && blk + 256 < n_blk) issue_sw(blk + 256 + 64 * wave);
        const uint32_t w_next = blk + 1 < n_blk ? sw_at(blk + 1) : w_cur;
        unsafe |= w_next;

        const int sv = blk_sv(w_cur);
        const bool solo = blk_new(blk);
        if (grp_n == kPfGroup || (grp_n > 0 && (solo || abs(grp_sv - sv) > 3))) {
            pf_flush(tl, static_cast<double>(pow2f(-grp_sv)));
            grp_n = 0;
        }
        if (grp_n == 0) grp_sv = sv;
        grp_n = solo ? kPfGroup : grp_n + 1;
        const float vshift = static_cast<float>(grp_sv - sv);

        uint32_t ph[2][2][4];
        f32x4_t snext[4];
        const uint8_t* knext = lds + kOffK + ((blk + 1) & 1) * kPlaneB;
        // The two waves of a SIMD run the same steps; the one in this MFMA + VALU mix gets
        // issue priority over the other's V^T P^T.
        __builtin_amdgcn_s_setprio(1);
        if (blk + 1 >= n_blk)
            pf_probs_and_next<false, false>(scur, mult_cur, vshift, knext, qop, n, g, tl, ph, snext);
        else if (blk_new(blk + 1))
            pf_probs_and_next<true, true>(scur, mult_cur, vshift, knext, qop, n, g, tl, ph, snext);
        else
            pf_probs_and_next<true, false>(scur, mult_cur, vshift, knext, qop, n, g, tl, ph, snext);
        __builtin_amdgcn_s_setprio(0);
        // fp16's subnormal quantum: a p below 2^-2 (in the units the MFMAs see) has a second part
        // below 2^-14, and the split carries it to within 2^-25 absolutely, not 2^-22 of itself
        // (a p below 2^-25 is dropped).  Harmless while those keys' V is about as large as the
        // rest's (what is lost is then below the calibrated rounding), not when keys of tiny
        // weight carry V far larger than the output.  So on blocks whose V is 2^6 times the
        // smallest-V block's or more (a uniform test), a lane with a p below 2^-2 among its 16
        // keys (the fp16 codes of the first parts, below 0x3400; masked keys count,
        // conservatively) adds their bound 16 * 2^-25 * 2^15 (staged |V| < 2^15) = 2^-6, times
        // 2^-grp_sv, to u, which the epilogue compares with the row's elements.
        if (grp_sv < sv_hi - 6) {
            uint32_t m16 = ph[0][0][0];
#pragma unroll
            for (int w = 0; w < 2; ++w)
#pragma unroll
                for (int d = 0; d < 4; ++d) m16 = pk_min_u16(m16, ph[0][w][d]);
            if (min(m16 & 0xffffu, m16 >> 16) < 0x3400u) tl.u += pow2f(-6 - grp_sv);
        }

        // The next block's running max is found before this block's V^T P^T (which still
        // accumulates at the current max); O and l move to it afterwards.
        const float mult_next = blk_mult(w_next);
        float m_next = tl.m_run;
        if (blk + 1 < n_blk)
            m_next = pf_next_max(snext, blk_diag(blk + 1), (blk + 1) * kPfBlk, g, pos_n, tl.m_run, mult_next);

        pf_pv(vaddr, (blk & 1) * kPlaneB, ph, tl);

        pf_rescale(tl, m_next);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) scur[kt] = snext[kt];
        w_cur = w_next;
        mult_cur = mult_next;
        // This wave's copies into LDS are complete; after the barrier every wave's are, and
        // every wave is done with the buffers the next step's copies go to.
        __builtin_amdgcn_s_waitcnt(0x0F70);    // vmcnt(0)
        __syncthreads();
    }
    pf_flush(tl, static_cast<double>(pow2f(-grp_sv)));

    double l = tl.l64 + __shfl_xor(tl.l64, 16);
    l += __shfl_xor(l, 32);
    float u = tl.u + __shfl_xor(tl.u, 16);
    u += __shfl_xor(u, 32);
    const double ul = static_cast<double>(u) / l;     // bound on that error in the row's elements
    // The row of query n: lanes n, n+16, n+32, n+48 hold dims 16dt + 4g ..
    double x[8][4];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) x[dt][i] = tl.o64[dt][i] / l;
    const bool q_bad_row = __shfl_xor(static_cast<int>(q_bad), 16) | __shfl_xor(static_cast<int>(q_bad), 32) |
                           __shfl_xor(static_cast<int>(q_bad), 48) | static_cast<int>(q_bad);
    const int64_t row = (static_cast<int64_t>(b) * T + tq_c) * kHq + hq;
    uint2 pk[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
        pk[dt].x = f32_to_bf16_out(static_cast<float>(x[dt][0])) |
                   (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(x[dt][1]))) << 16);
        pk[dt].y = f32_to_bf16_out(static_cast<float>(x[dt][2])) |
                   (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(x[dt][3]))) << 16);
    }
    // The rescore flag, decided here from the rounded row: rows that read a marked block or
    // whose Q row is out of range always go to the rescore.  Waves past the last query (q_ok
    // false in every lane) decide nothing.
    if (a.rs_hdr && __ballot(q_ok)) {
        const bool forced = (unsafe >> 31) != 0u || q_bad_row;
        if (pf_flag_row(a, b, kvh, st, st + tq_c, row, tl.m_run, forced, ul, pk, lane) && q_ok && g == 0)
            rs_append(a, static_cast<uint32_t>(row));
    }
    if (!q_ok) return;
    uint16_t* orow = a.out + row * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * g) = pk[dt];
}

hipError_t launch_prefill_attention(const PrefillArgs& a, hipStream_t stream) {
    const int64_t n_wg = static_cast<int64_t>(a.batch) * kHkv * a.n_qblk;
    if (n_wg == 0) return hipSuccess;
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(static_cast<unsigned>(n_wg)), dim3(kPfThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace gqa

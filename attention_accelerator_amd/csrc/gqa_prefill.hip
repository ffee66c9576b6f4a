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
// rows of each 64-key block are loaded once per workgroup into LDS and used by all 4
// heads of the group and all 32 positions (gqa_kv_broadcast.v:38-59 at block scale).
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
#include "gqa_device.h"
#include "gqa_internal.h"

namespace gqa {

namespace {

constexpr int kPfPos = 32;                 // query positions per workgroup
constexpr int kPfWaves = 8;                // 4 Q heads x 2 tiles of 16 positions
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfBlk = 64;                 // keys per K/V block

constexpr uint32_t kPermLo = 0x05040100u;  // v_perm_b32: low halves of (b, a) -> a.lo | b.lo << 16
constexpr uint32_t kPermHi = 0x07060302u;  // high halves

}  // namespace

// The second and third BF16 parts of every rotated new K row, then one zero row (the parts
// of a cached key, which the attention kernel copies for keys before the chunk).
size_t prefill_split_bytes(int32_t batch, int32_t n_new) {
    return (2ull * static_cast<size_t>(batch) * static_cast<size_t>(n_new) * kHkv + 1) * kD * sizeof(uint16_t);
}

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
    if (rope) rope_sincos(pos, a.rope.inv_freq[lane], sn, cs);
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

// LDS holds two blocks (double buffer), each: K (the cache row, plane 0), the second and
// third BF16 parts of chunk keys (planes 1, 2) and V, 64 rows of 256 B per plane (128 KB in
// all).  Rows are copied from HBM straight into LDS (global_load_lds_dwordx4: lane l of an
// instruction writes bytes [16l, 16l + 16) of a 1 KB stretch = 4 rows), so a row's 16
// 16-byte chunks are placed by choosing which chunk each lane fetches: chunk c of row r
// sits at position c ^ pf_swz(r).  With that swizzle the K operand reads (16 rows, one
// chunk) and the V^T transpose reads (16 rows, two chunks) hit 64 distinct banks per
// half-wave.
constexpr int kRowB = 256;                  // LDS bytes per row
constexpr int kPlaneB = kPfBlk * kRowB;     // 16 KB per plane
constexpr int kBufB = 4 * kPlaneB;          // K, K part 2, K part 3, V
constexpr int kVOff = 3 * kPlaneB;

__device__ __forceinline__ int pf_swz(int row) { return (2 * row + (row >> 3)) & 15; }

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// Request block blk into the LDS buffer at `dst`.  Wave w fetches rows
// 8w .. 8w+7 (two 4-row instructions per plane).  Rows past the keys this workgroup needs
// repeat its last key; planes 1 and 2 are fetched only for a block holding chunk keys, and a
// cached key's parts come from the zero row.
__device__ __forceinline__ void pf_issue_block(const PrefillArgs& a, const char* kbase, const char* vbase,
                                               int b, int kvh, int st, int blk, int n_keys, bool has_new,
                                               uint8_t* dst, int wave, int lane) {
    const int key0 = blk * kPfBlk;
    const int64_t row_bytes = a.kv_pos_stride * 2;
    const int64_t n_rows = static_cast<int64_t>(a.batch) * a.n_new * kHkv;
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int r = 4 * (2 * wave + ii) + (lane >> 4);
        const int c = (lane & 15) ^ pf_swz(r);
        const int key = min(key0 + r, n_keys - 1);
        const int stretch = (2 * wave + ii) * 1024;
        const int64_t off = static_cast<int64_t>(key) * row_bytes + 16 * c;
        __builtin_amdgcn_global_load_lds(kbase + off, (lds_void_t*)(dst + stretch), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vbase + off, (lds_void_t*)(dst + kVOff + stretch), 16, 0, 0);
        if (has_new) {
            const int u = key - st;          // chunk row of this key (< 0: a cached key)
            const int64_t prow = u < 0 ? 2 * n_rows : (static_cast<int64_t>(b) * a.n_new + u) * kHkv + kvh;
            const int64_t lrow = u < 0 ? 2 * n_rows : n_rows + prow;
            const char* p1 = reinterpret_cast<const char*>(a.k_split + prow * kD) + 16 * c;
            const char* p2 = reinterpret_cast<const char*>(a.k_split + lrow * kD) + 16 * c;
            __builtin_amdgcn_global_load_lds(p1, (lds_void_t*)(dst + kPlaneB + stretch), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(p2, (lds_void_t*)(dst + 2 * kPlaneB + stretch), 16, 0, 0);
        }
    }
}

// 8 K values of row `row`, bytes [16 chunk, 16 chunk + 16) of the plane at `plane`.
__device__ __forceinline__ bf16x8_t pf_k_chunk(const uint8_t* plane, int row, int chunk) {
    return *reinterpret_cast<const bf16x8_t*>(plane + row * kRowB + 16 * (chunk ^ pf_swz(row)));
}

// V^T operand of the 32-key window w, dims 16dt .. 16dt+15: lane (g, m) gets keys
// 32w + 4g + i (slots 0..3) and 32w + 16 + 4g + i (slots 4..7) of dim 16dt + m, through two
// transpose reads (ds_read_b64_tr_b16: lane i of a 16-lane group receives element i%4 of
// the 8 bytes addressed by lane 4j + i/4, j = 0..3).  Supplying lane a addresses row
// 32w + 4g + a/4 (+16), dims 16dt + 4(a%4) .. +3.
__device__ __forceinline__ bf16x8_t pf_vt_operand(const uint8_t* vplane, int w, int dt, int lane) {
    const int g = lane >> 4;
    const int a = lane & 15;
    const int row = 32 * w + 4 * g + (a >> 2);
    const int chunk = 2 * dt + ((a & 3) >> 1);
    const int half = (a & 1) * 8;
    const uint8_t* p0 = vplane + row * kRowB + 16 * (chunk ^ pf_swz(row)) + half;
    const uint8_t* p1 = vplane + (row + 16) * kRowB + 16 * (chunk ^ pf_swz(row + 16)) + half;
    const short4_t r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4_t*)(p0));
    const short4_t r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4_t*)(p1));
    union {
        short4_t h[2];
        bf16x8_t v;
    } u;
    u.h[0] = r0;
    u.h[1] = r1;
    return u.v;
}

// Upper 16 bits of two floats packed as BF16 codes (truncation; used for exact splits).
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), kPermHi);
}

// Scores S^T[key][query] of one 16-query tile over the block's 4 key tiles: the 3 BF16 parts
// of Q against the cache row, and for chunk keys the (k2,q1), (k2,q2), (k3,q1) products.
template <bool kNew>
__device__ __forceinline__ void pf_scores(const uint8_t* kp, const bf16x8_t (&qop)[3][4], int n, int g,
                                          f32x4_t (&sacc)[4]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) sacc[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        bf16x8_t ak[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k_chunk(kp, 16 * kt + n, 4 * kb + g);
#pragma unroll
        for (int s = 0; s < 3; ++s)
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
                sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[kt], qop[s][kb], sacc[kt], 0, 0, 0);
        if (kNew) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k_chunk(kp + kPlaneB, 16 * kt + n, 4 * kb + g);
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
                    sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[kt], qop[s][kb], sacc[kt], 0, 0, 0);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) ak[kt] = pf_k_chunk(kp + 2 * kPlaneB, 16 * kt + n, 4 * kb + g);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
                sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[kt], qop[0][kb], sacc[kt], 0, 0, 0);
        }
    }
}

// Per-tile softmax state: the running max (integer-valued, log2 units), sum and O (fp64,
// lane (g, n): O^T[16dt + 4g + i][query n]).
struct PfTile {
    double o64[8][4];
    double l64;
    float m_run;
};

// Block max of a tile's scores (masking keys past each query on diagonal blocks); grows the
// running max to ceil(block max) and rescales O and l by the exact power of two.
__device__ __forceinline__ void pf_block_max(f32x4_t (&sacc)[4], bool diag, int key0, int g, int pos_n, PfTile& t) {
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
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    const bool grow = bmax > t.m_run;
    if (__ballot(grow)) {
        const float m_new = grow ? ceilf(bmax) : t.m_run;
        const int shift = (t.m_run == -INFINITY) ? 0 : static_cast<int>(t.m_run - m_new);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) t.o64[dt][i] = ldexp(t.o64[dt][i], shift);
        t.l64 = ldexp(t.l64, shift);
        t.m_run = m_new;
    }
}

// p = 2^(s - m) (0 for masked keys), summed into l, split by truncation into three BF16
// parts packed as the P^T B operand: ph[part][window][dword].
__device__ __forceinline__ void pf_probs(const f32x4_t (&sacc)[4], PfTile& t, uint32_t (&ph)[3][2][4]) {
    float lsum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
        float p[4], r1[4], r2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // v_exp_f32: 2^x, 0 for -inf (masked keys); results below 2^-126 flush to 0,
            // far below anything the BF16 output can see.
            p[i] = __builtin_amdgcn_exp2f(sacc[kt][i] - t.m_run);
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
    t.l64 += static_cast<double>(lsum);
}

// O^T[dim][query] += the block's V^T P^T: per 16-dim tile, V^T (transpose reads) against the
// three P parts of both 32-key windows in fp32, then added into the fp64 O; two tiles at a
// time, so that few accumulators are live.
__device__ __forceinline__ void pf_pv(const uint8_t* vp, const uint32_t (&ph)[3][2][4], int lane, PfTile& t) {
    bf16x8_t pb[2][3];
#pragma unroll
    for (int w = 0; w < 2; ++w)
#pragma unroll
        for (int s = 0; s < 3; ++s) pb[w][s] = as_bf16x8(make_uint4(ph[s][w][0], ph[s][w][1], ph[s][w][2], ph[s][w][3]));
#pragma unroll
    for (int d0 = 0; d0 < 8; d0 += 2) {
        f32x4_t oacc[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) oacc[e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const bf16x8_t av = pf_vt_operand(vp, w, d0 + e, lane);
#pragma unroll
                for (int s = 0; s < 3; ++s)
                    oacc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[w][s], oacc[e], 0, 0, 0);
            }
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) t.o64[d0 + e][i] += static_cast<double>(oacc[e][i]);
    }
}

__global__ __launch_bounds__(kPfThreads) void prefill_attn_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kBufB];

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

    const int tq_c = min(tq, T - 1);
    const int pos_n = st + tq_c;            // this lane's query position
    const bool wave_has_q = t_wave0 < T;
    const int n_keys = st + min(T, qb * kPfPos + kPfPos);
    const int n_keys_wave = st + min(T, t_wave0 + 16);
    const int n_blk = (n_keys + kPfBlk - 1) / kPfBlk;
    const int64_t head_elem = static_cast<int64_t>(b) * a.kv_batch_stride +
                              static_cast<int64_t>(kvh) * a.kv_head_stride;
    const char* kbase = reinterpret_cast<const char*>(a.k + head_elem);
    const char* vbase = reinterpret_cast<const char*>(a.v + head_elem);

    // Block 0 is requested before the Q operands are formed.
    pf_issue_block(a, kbase, vbase, b, kvh, st, 0, n_keys, kPfBlk - 1 >= st, lds, wave, lane);

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

    PfTile tl;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) tl.o64[dt][i] = 0.0;
    tl.l64 = 0.0;
    tl.m_run = -INFINITY;

    for (int blk = 0; blk < n_blk; ++blk) {
        // This wave's copies into LDS are complete; after the barrier every wave's are, and
        // every wave is done with the buffer the next block goes to.
        __builtin_amdgcn_s_waitcnt(0x0F70);    // vmcnt(0)
        __syncthreads();
        if (blk + 1 < n_blk) {
            const int nb = blk + 1;
            pf_issue_block(a, kbase, vbase, b, kvh, st, nb, n_keys, nb * kPfBlk + kPfBlk - 1 >= st,
                           lds + (nb & 1) * kBufB, wave, lane);
        }
        const int key0 = blk * kPfBlk;
        if (!wave_has_q || key0 >= n_keys_wave) continue;
        const uint8_t* kp = lds + (blk & 1) * kBufB;
        f32x4_t sacc[4];
        if (key0 + kPfBlk - 1 >= st)
            pf_scores<true>(kp, qop, n, g, sacc);
        else
            pf_scores<false>(kp, qop, n, g, sacc);
        pf_block_max(sacc, key0 + kPfBlk - 1 > st + t_wave0, key0, g, pos_n, tl);
        uint32_t ph[3][2][4];
        pf_probs(sacc, tl, ph);
        pf_pv(kp + kVOff, ph, lane, tl);
    }

    if (!q_ok) return;
    double l = tl.l64 + __shfl_xor(tl.l64, 16);
    l += __shfl_xor(l, 32);
    uint16_t* orow = a.out + ((static_cast<int64_t>(b) * T + tq) * kHq + hq) * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
        uint2 pk;
        pk.x = f32_to_bf16_rne(static_cast<float>(tl.o64[dt][0] / l)) |
               (static_cast<uint32_t>(f32_to_bf16_rne(static_cast<float>(tl.o64[dt][1] / l))) << 16);
        pk.y = f32_to_bf16_rne(static_cast<float>(tl.o64[dt][2] / l)) |
               (static_cast<uint32_t>(f32_to_bf16_rne(static_cast<float>(tl.o64[dt][3] / l))) << 16);
        *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * g) = pk;
    }
}

hipError_t launch_prefill_attention(const PrefillArgs& a, hipStream_t stream) {
    const int64_t n_wg = static_cast<int64_t>(a.batch) * kHkv * a.n_qblk;
    if (n_wg == 0) return hipSuccess;
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(static_cast<unsigned>(n_wg)), dim3(kPfThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace gqa

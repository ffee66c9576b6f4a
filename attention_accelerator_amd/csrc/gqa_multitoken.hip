// gqa_multitoken.hip -- multi-token decode for gfx950: chunks of at most 16 new tokens per
// sequence (draft verification, a few decode steps at once) split stream-K over all CUs
// with the prefill kernel's arithmetic (gqa_prefill.hip); the golden step per token is
// pyfiles/gen_gqa_wrapper_vectors.py:121-139 at query position start + t.
#include "gqa_device.h"
#include "gqa_internal.h"
#include "gqa_prefill_common.h"
#include "gqa_streamk.h"

namespace gqa {

// ---------------------------------------------------------------------------------
// Multi-token decode: chunks of at most kMultiMaxNew (16) new tokens per sequence --
// drafted tokens being verified, or decode steps that append their own K/V.  The prefill
// attention kernel (gqa_prefill.hip) gives each (sequence, KV head, 32 positions) one workgroup over all of that
// sequence's keys, which for a short chunk leaves most of its MFMA columns empty and a
// ragged batch waiting for its longest sequence.  Here the query rows of a KV head's group
// form MFMA B operands of 16 columns -- tile w holds tokens 4w .. 4w+3 of the 4 heads,
// column 16w + n for token 4w + n/4 and head n%4 -- and the keys are split stream-K as in
// the decode path: every segment (sequence, KV head) holds start + T keys, a range's part
// of a segment is a piece, a split segment's pieces leave partials that mt_merge_kernel
// combines.  The arithmetic is the attention kernel's: three BF16 parts of Q, the chunk's
// own keys at full precision, P in three parts, fp64 accumulation within a piece (fp32
// partials between pieces), integer-valued running max.
//
// A workgroup has one wave per column tile (W = 1, 2 or 4 waves for T <= 4, 8 or 16).  With
// one tile (HBM-bound) there is one wave per SIMD, 4 * CUs workgroups; with two or four
// tiles every window costs each wave about 2,000 cycles of MFMA and fp64 work, and two waves
// per SIMD (8 * CUs / W workgroups) let one wave's MFMA run beside the other's VALU work.
// Per 32-key window the workgroup copies the window's K rows and V rows (a plane of 8 KB
// each) from HBM into LDS once -- each wave issues 8/W of the plane's 1 KB copies -- and
// every wave forms its tile's scores and V^T P^T from them.  The planes form a ring in the
// order K0 V0 K1 V1 ...: while window i is computed, K of windows i+1 .. i+A+1 and V of
// windows i+1 .. i+A are in flight.  A = 1 (2A + 3 = 5 slots, 40 KB per workgroup) keeps 12
// planes in flight per CU with four one- or two-wave workgroups, 6 with two four-wave ones
// (measured: A = 1, 2, 3 for W = 4 within 1 %, A = 1 fastest).
//
// Each wave forms the next window's scores beside the current window's probabilities.
// It waits for its own copies, then a fence-free barrier makes the whole plane visible:
// once per window after the next window's K lands (which also tells every wave that V of
// the previous window has been read, so its slot may be refilled; and since each wave
// requested the current window's V before that K, V has landed too).  Only a piece's last
// window, which waits for no next K, waits and meets again for its V.

constexpr int kMtWin = 32;                    // keys per window
constexpr int kMtPlaneB = kMtWin * kRowB;     // 8 KB: 32 rows of 256 B
constexpr int kMtTile = 16;                   // query rows per wave: 4 heads x 4 tokens
constexpr int kMtCopies = kMtWin / 4;         // 1 KB copies per plane (each writes 4 rows)
// Stream positions charged per segment start: a piece here costs more than in decode (the
// Q operands, the fp32 partial of 16W columns), about two windows' streaming time for one
// tile and more for two or four (their workgroups share a SIMD).  Measured on B=64 ragged:
// W = 1 best at 64 of 32, 48, 64, 96 (T=4 216.5 -> 215.4 us); W = 2 and 4 best at 128 of 32,
// 64, 128, 192 (T=8 248.7 -> 246.9 us, T=16 374.6 -> 370.8 us).
__host__ __device__ constexpr int mt_seg_lead(int w) { return w == 1 ? 64 : 128; }

__host__ __device__ constexpr int mt_ahead(int) { return 1; }
__host__ __device__ constexpr int mt_slots(int w) { return 2 * mt_ahead(w) + 3; }

// s_waitcnt immediate for vmcnt(n) alone (gfx9: vmcnt bits 3:0 and 15:14, expcnt and
// lgkmcnt at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
static_assert(vmcnt_imm(0) == 0x0F70 && vmcnt_imm(16) == 0x4F70, "vmcnt encoding");

// Wait until at most kPlanes planes of this wave's copies (kC instructions each) are in
// flight -- the count when the producer runs its full kA windows ahead (`steady`) -- and
// otherwise until none is: the counter retires in issue order, so everything older has
// landed.  Only a range's last kA windows, where nothing is left to overlap, take the full
// wait (a switch over the exact count cost ~20 scalar instructions and ~8 branches per
// window).  Requests of other kinds issued since (Q operands, stores) only make the wait
// longer.
template <int kC, int kPlanes>
__device__ __forceinline__ void mt_wait_planes(bool steady) {
    static_assert(kPlanes * kC <= 63, "vmcnt range");
    if (steady)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kPlanes * kC));
    else
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

// Barrier without the memory fence __syncthreads adds (which would wait for every copy in
// flight).
__device__ __forceinline__ void mt_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Barrier after this wave's LDS writes have completed, without waiting for its global stores
// (which nothing after the barrier reads).
__device__ __forceinline__ void mt_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

int32_t multi_waves(int32_t n_new) { return n_new <= 4 ? 1 : n_new <= 8 ? 2 : 4; }
int32_t multi_simd_waves(int32_t n_new) { return n_new <= 4 ? 1 : 2; }

// Keys of sequence b's segments: every key its last new token sees (0 for a start outside
// [0, capacity - T]).
__device__ __forceinline__ int mt_keys(const PrefillArgs& a, int b) {
    const int st = a.start[b];
    return prefill_start_ok(a, st) ? st + a.n_new : 0;
}

namespace {
struct MtLayout {
    size_t q_op, plan, seq_off, part_o, part_ml, chunk_s, piece_st, total;
};

MtLayout mt_layout(int32_t batch, int32_t n_new, int32_t n_wgs) {
    const size_t w = static_cast<size_t>(multi_waves(n_new));
    const size_t cols = kMtTile * w;
    const size_t n_slots = static_cast<size_t>(n_wgs) + static_cast<size_t>(kHkv) * batch;
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    MtLayout l{};
    l.q_op = 0;
    l.plan = l.q_op + al(static_cast<size_t>(batch) * kHkv * w * 8 * kWave * sizeof(float4));
    l.seq_off = l.plan + 256;
    l.part_o = l.seq_off + al((static_cast<size_t>(batch) + 1) * sizeof(int64_t));
    l.part_ml = l.part_o + al(n_slots * cols * kD * sizeof(float));
    l.chunk_s = l.part_ml + al(n_slots * cols * sizeof(float2));
    l.piece_st = l.chunk_s + al(static_cast<size_t>(batch) * kHkv * cols * 4 * w * sizeof(float));
    l.total = l.piece_st + al(n_slots * w * (8 + kD) * sizeof(uint32_t));
    return l;
}
}  // namespace

size_t prefill_multi_bytes(int32_t batch, int32_t n_new, int32_t n_wgs) {
    return mt_layout(batch, n_new, n_wgs).total;
}

void prefill_multi_layout(PrefillArgs& a, void* base, int32_t n_wgs) {
    const MtLayout l = mt_layout(a.batch, a.n_new, n_wgs);
    char* p = static_cast<char*>(base);
    a.q_op = reinterpret_cast<float4*>(p + l.q_op);
    a.plan_hdr = reinterpret_cast<int64_t*>(p + l.plan);
    a.seq_off = reinterpret_cast<int64_t*>(p + l.seq_off);
    a.part_o = reinterpret_cast<float*>(p + l.part_o);
    a.part_ml = reinterpret_cast<float2*>(p + l.part_ml);
    a.chunk_s = reinterpret_cast<float*>(p + l.chunk_s);
    a.piece_st = reinterpret_cast<uint32_t*>(p + l.piece_st);
    a.n_wgs = n_wgs;
}

// The stream-K plan (one wave): seq_off[b] = stream position of sequence b's first segment,
// seq_off[B] = total, header {total, positions per workgroup, lead, XCD extra}
// (gqa_streamk.h).
template <int kW>
__device__ __forceinline__ void mt_build_plan(const PrefillArgs& a, int lane) {
    int64_t sum = 0;
    int max_keys = 0, n_seq = 0;
    // The first 64 sequences' keys are kept for the scan below (the header stores between
    // the two passes would otherwise make the compiler load them again).
    const int k_first = lane < a.batch ? mt_keys(a, lane) : 0;
    for (int base = 0; base < a.batch; base += kWave) {
        const int b = base + lane;
        const int k = base == 0 ? k_first : (b < a.batch ? mt_keys(a, b) : 0);
        sum += wave_sum_i64(k);
        max_keys = max(max_keys, static_cast<int>(wave_max_i64(k)));
        n_seq += static_cast<int>(wave_sum_i64(k > 0 ? 1 : 0));
    }
    int lead;
    int64_t total, per_wg;
    plan_lead_totals(sum, max_keys, n_seq, a.n_wgs, lead, total, per_wg, mt_seg_lead(kW));
    if (lane == 0) {
        a.plan_hdr[0] = total;
        a.plan_hdr[1] = per_wg;
        a.plan_hdr[2] = lead;
        a.plan_hdr[3] = range_extra(per_wg, a.skew_pm);
        a.seq_off[a.batch] = total;
    }
    int64_t carry = 0;
    for (int base = 0; base < a.batch; base += kWave) {
        const int b = base + lane;
        const int k = base == 0 ? k_first : (b < a.batch ? mt_keys(a, b) : 0);
        const int span = k > 0 ? k + lead : 0;
        const int64_t incl = wave_incl_scan_i64(span, lane) + carry;
        if (b < a.batch) a.seq_off[b] = (incl - span) * kHkv;
        carry = __shfl(incl, kWave - 1);
    }
}

// Four consecutive BF16 values from p: one 8-byte load when the tensor is 16-byte aligned
// (kVec; p is then a multiple of 4 elements past an aligned row start), else four 2-byte
// loads.
template <bool kVec>
__device__ __forceinline__ void load4(const uint16_t* p, uint16_t (&h)[4]) {
    if (kVec) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        h[0] = static_cast<uint16_t>(v.x & 0xFFFFu);
        h[1] = static_cast<uint16_t>(v.x >> 16);
        h[2] = static_cast<uint16_t>(v.y & 0xFFFFu);
        h[3] = static_cast<uint16_t>(v.y >> 16);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i] = p[i];
    }
}

// Per (sequence b, KV head kvh), four waves; wave w:
//  - the KV append of this head's new rows u = w, w + 4, ... (what kv_append_kernel does
//    for all heads): lane i rotates the pair (i, i + 64) at position start + u in double
//    and writes it rounded to BF16, and copies the V row;
//  - a quarter of the Q operands of every column tile: lane (g, n) of tile tau holds
//    column 16 tau + n (token 4 tau + n/4, Q head 4*kvh + n%4) at dims 32kb + 8g + j; wave
//    w takes kb = w & 1 and its pair kb + 2, j in [4(w >> 1), +4), rotated at the token's
//    position and scaled by scale*log2(e) in double, stored rounded to f32 (the stream
//    kernel splits each into three BF16 parts, exactly); columns of tokens t >= T are zero;
//  - the same dims' share of the scores of the chunk's own keys (key start + u, u < T:
//    the new K row rotated at its position and not rounded, as the reference rotates K)
//    against every column, in double (fp64 MFMAs).  The four shares are added in a fixed
//    order and rounded once to f32: the stream kernel takes these scores in place of the
//    ones it would form from the cache's rounded copy of those rows.
// Row B of the grid builds the plan.  A sequence whose start is out of range gets NaN
// rows and no cache write.
template <bool kVec, int kW>
__global__ __launch_bounds__(256) void mt_prepare_kernel(PrefillArgs a) {
    constexpr int kCols = kMtTile * kW;
    constexpr int kU = 4 * kW;                // chunk keys per column held (>= T)
    const int kvh = blockIdx.x;
    const int b = blockIdx.y;
    const int w = threadIdx.x >> 6;
    const int lane = threadIdx.x & (kWave - 1);
    if (b == a.batch) {
        if (kvh == 0 && w == 0) mt_build_plan<kW>(a, lane);
        if (kvh == 1) rs_clear(a, threadIdx.x);
        return;
    }
    const int T = a.n_new;
    const int st = a.start[b];
    // Every load before any store or barrier (a store may alias them as far as the compiler
    // knows, and a load placed after it or after the barrier would wait for it): the append
    // rows, Q, and the chunk's K rows at this lane's dims.
    const int g = lane >> 4;
    const int n = lane & 15;
    const int kbp = w & 1;
    const int d0 = 32 * kbp + 8 * g + 4 * (w >> 1);
    uint16_t akx[kW], aky[kW], avx[kW], avy[kW];
#pragma unroll
    for (int r = 0; r < kW; ++r) {
        const int u = w + 4 * r;
        akx[r] = aky[r] = avx[r] = avy[r] = 0;
        if (u < T) {
            const int64_t row = ((static_cast<int64_t>(b) * T + u) * kHkv + kvh) * kD;
            akx[r] = a.k_new[row + lane];
            aky[r] = a.k_new[row + lane + kPairs];
            avx[r] = a.v_new[row + lane];
            avy[r] = a.v_new[row + lane + kPairs];
        }
    }
    uint16_t qx[kW][4], qy[kW][4];
#pragma unroll
    for (int tau = 0; tau < kW; ++tau) {
        const int tc = min(4 * tau + (n >> 2), T - 1);
        const uint16_t* qrow = a.q + ((static_cast<int64_t>(b) * T + tc) * kHq + kvh * kGroup + (n & 3)) * kD;
        load4<kVec>(qrow + d0, qx[tau]);
        load4<kVec>(qrow + d0 + kPairs, qy[tau]);
    }
    // The chunk key u = n of this lane's rows of the fp64 score MFMAs.
    uint16_t kxh[4] = {0, 0, 0, 0}, kyh[4] = {0, 0, 0, 0};
    if (n < T) {
        const uint16_t* krow = a.k_new + ((static_cast<int64_t>(b) * T + n) * kHkv + kvh) * kD;
        load4<kVec>(krow + d0, kxh);
        load4<kVec>(krow + d0 + kPairs, kyh);
    }
    // The rescore's counters start at zero (also for a sequence whose start is out of range:
    // the tile counters are indexed by tile, not by row).
    if (a.rs_hdr) {
        for (int i = threadIdx.x; i < T * kGroup; i += blockDim.x)
            a.rs_done[(static_cast<int64_t>(b) * T + i / kGroup) * kHq + kvh * kGroup + i % kGroup] = 0u;
        if (threadIdx.x == 0) a.rs_gcnt[b * kHkv + kvh] = 0u;
    }
    if (!prefill_start_ok(a, st)) {
        for (int i = threadIdx.x; i < T * kGroup * (kD / 4); i += blockDim.x) {
            const int tt = i / (kGroup * (kD / 4));
            const int r = i % (kGroup * (kD / 4));
            uint2* o = reinterpret_cast<uint2*>(a.out + ((static_cast<int64_t>(b) * T + tt) * kHq + kvh * kGroup) * kD);
            o[r] = make_uint2(0x7fc07fc0u, 0x7fc07fc0u);
        }
        return;
    }
    // sin and cos of (start + u) * inv_freq[i]: wave u % 4, lane i.
    __shared__ double sn_s[kU][kPairs], cs_s[kU][kPairs];
    // Row u of a wave's share padded by one double, so that the final pass (consecutive
    // threads, consecutive u) reads distinct banks.
    __shared__ double part_s[4][kU][kCols + 1];
    // The chunk rows' statistics for the rescore flag: squared pair-group norms of the rotated
    // K rows (fp32 bits) and |V| codes, per token.
    __shared__ uint32_t kn_s[kU][8];
    __shared__ uint16_t vd_s[kU][kD];
    const bool rope_q = (a.flags & 1u) != 0;
    const bool rope_k = (a.flags & 2u) != 0;
    if (rope_q || rope_k)
#pragma unroll
        for (int r = 0; r < kW; ++r) {       // unrolled: the sincos chains of one lane overlap
            const int u = w + 4 * r;
            if (u < T) {
                rope_sincos(static_cast<int64_t>(st) + u, a.rope.inv_freq[lane], sn_s[u][lane], cs_s[u][lane]);
                if (kvh == 0 && a.rs_hdr)
                    a.rs_cs[(static_cast<int64_t>(b) * T + u) * kPairs + lane] = make_double2(cs_s[u][lane], sn_s[u][lane]);
            }
        }
    mt_lds_barrier();

    double qvx[kW][4], qvy[kW][4];
#pragma unroll
    for (int tau = 0; tau < kW; ++tau) {
        const int t = 4 * tau + (n >> 2);
        const bool col = t < T;
        const int tc = col ? t : T - 1;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int d = d0 + jj;
            const double x = bf16_to_f32(qx[tau][jj]);
            const double y = bf16_to_f32(qy[tau][jj]);
            double xr = x, yr = y;
            if (rope_q) {
                const double sn = sn_s[tc][d], cs = cs_s[tc][d];
                xr = x * cs - y * sn;
                yr = x * sn + y * cs;
            }
            qvx[tau][jj] = col ? xr * a.qk_scale_log2 : 0.0;
            qvy[tau][jj] = col ? yr * a.qk_scale_log2 : 0.0;
        }
    }
    // This wave's share of the chunk-key scores: per tile, S[u][column] over this wave's 32
    // dims by fp64 MFMAs (v_mfma_f64_16x16x4: A[u][k] in lane 16k + u, B[k][column] in lane
    // 16k + column, D[k + 4r][column] in lane 16k + column, register r), the k index of step
    // (half, jj) standing for dim d0(k) + jj + 64 half -- the same dims the lane holds as Q
    // operands.  Rows u >= T are zero; a row the causal mask hides from a column (u > 4 tau
    // + 3) is never read.
    {
        double kxr[4], kyr[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const double x = bf16_to_f32(kxh[jj]);
            const double y = bf16_to_f32(kyh[jj]);
            kxr[jj] = x;
            kyr[jj] = y;
            if (rope_k && n < T) {
                const double sn = sn_s[n][d0 + jj], cs = cs_s[n][d0 + jj];
                kxr[jj] = x * cs - y * sn;
                kyr[jj] = x * sn + y * cs;
            }
        }
#pragma unroll
        for (int tau = 0; tau < kW; ++tau) {
            f64x4_t acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(kxr[jj], qvx[tau][jj], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(kyr[jj], qvy[tau][jj], acc, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (g + 4 * r < kU) part_s[w][g + 4 * r][kMtTile * tau + n] = acc[r];
        }
    }

    // Stores: the appended cache rows, this wave's quarter of the Q operands.
#pragma unroll
    for (int r = 0; r < kW; ++r) {
        const int u = w + 4 * r;
        if (u < T) {
            const int64_t ce = cache_elem(a, b, kvh, static_cast<int64_t>(st) + u);
            double xr = bf16_to_f32(akx[r]), yr = bf16_to_f32(aky[r]);
            if (rope_k) {
                const double x = xr, y = yr;
                xr = x * cs_s[u][lane] - y * sn_s[u][lane];
                yr = x * sn_s[u][lane] + y * cs_s[u][lane];
            }
            if (ce >= 0) {
                a.k[ce + lane] = bf16_of(xr);
                a.k[ce + lane + kPairs] = bf16_of(yr);
                a.v[ce + lane] = avx[r];
                a.v[ce + lane + kPairs] = avy[r];
            }
            if (a.rs_hdr) {
                // Lane i holds pair i of the row: its group is i / 8.
                float sq = static_cast<float>(xr * xr + yr * yr);
                sq += __shfl_xor(sq, 1);
                sq += __shfl_xor(sq, 2);
                sq += __shfl_xor(sq, 4);
                if ((lane & 7) == 0) kn_s[u][lane >> 3] = __float_as_uint(sq);
                vd_s[u][lane] = avx[r] & 0x7fffu;
                vd_s[u][lane + kPairs] = avy[r] & 0x7fffu;
            }
        }
    }
#pragma unroll
    for (int tau = 0; tau < kW; ++tau) {
        // float4 f = 2 kb + h of lane (g, n) holds dims 32 kb + 8 g + 4 h .. +3.
        float4* base = a.q_op + ((static_cast<int64_t>(b) * kHkv + kvh) * kW + tau) * 8 * kWave + lane;
        base[(2 * kbp + (w >> 1)) * kWave] =
            make_float4(static_cast<float>(qvx[tau][0]), static_cast<float>(qvx[tau][1]),
                        static_cast<float>(qvx[tau][2]), static_cast<float>(qvx[tau][3]));
        base[(2 * (kbp + 2) + (w >> 1)) * kWave] =
            make_float4(static_cast<float>(qvy[tau][0]), static_cast<float>(qvy[tau][1]),
                        static_cast<float>(qvy[tau][2]), static_cast<float>(qvy[tau][3]));
    }
    mt_lds_barrier();
    if (a.rs_hdr && threadIdx.x < 8 + kD) {
        // Running maxima over the chunk's tokens (rescore flag: token t sees chunk keys <= t),
        // and the cached-key maxima of this segment cleared for the stream kernel.
        const int64_t bh = static_cast<int64_t>(b) * kHkv + kvh;
        const int c = threadIdx.x;
        // Unrolled over the most tokens a tile set holds, every LDS read issued up front.
        uint32_t x[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) x[u] = u < T ? (c < 8 ? kn_s[u][c] : static_cast<uint32_t>(vd_s[u][c - 8])) : 0u;
        uint32_t run = 0u;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            run = max(run, x[u]);
            if (u < T) {
                if (c < 8)
                    a.rs_kpre[(bh * T + u) * 8 + c] = run;
                else
                    a.rs_dpre[(bh * T + u) * kD + c - 8] = static_cast<uint16_t>(run);
            }
        }
    }
    float* cs_out = a.chunk_s + (static_cast<int64_t>(b) * kHkv + kvh) * kCols * kU;
    for (int i = threadIdx.x; i < kCols * kU; i += blockDim.x) {
        const int c = i / kU;
        const int u = i % kU;
        cs_out[i] = static_cast<float>(((part_s[0][u][c] + part_s[1][u][c]) + part_s[2][u][c]) + part_s[3][u][c]);
    }
}

// This wave's share (copies [wv * kC, (wv + 1) * kC)) of one plane: K or V rows of the
// window of keys [key0, key0 + 32) of a segment (rows past k_last repeat row k_last), into
// the ring slot at `dst`, nontemporal (each row is read once): lane l of copy ii writes row
// 4ii + l/16, chunk position l%16, the chunk it fetches swizzled as in the attention
// kernel.
template <int kC>
__device__ __forceinline__ void mt_issue_plane(const char* seg, int64_t row_bytes, int key0, int k_last,
                                               uint8_t* dst, int wv, int lane) {
    constexpr int kNt = 2;     // cache policy: nontemporal
    if (key0 + kMtWin - 1 <= k_last) {
        // Every row of the window exists: a uniform row base plus the lane's 32-bit offset,
        // which does not change from window to window (the ABI keeps a (sequence, KV head)'s
        // rows under 4 GiB).
        const char* base = seg + static_cast<uint32_t>(key0) * static_cast<uint32_t>(row_bytes);
#pragma unroll
        for (int q = 0; q < kC; ++q) {
            const uint32_t r = static_cast<uint32_t>(4 * (wv * kC + q) + (lane >> 4));
            const uint32_t o = r * static_cast<uint32_t>(row_bytes) + 16u * static_cast<uint32_t>((lane & 15) ^ pf_swz(r));
            __builtin_amdgcn_global_load_lds(base + o, (lds_void_t*)(dst + (wv * kC + q) * 1024), 16, 0, kNt);
        }
        return;
    }
    int64_t off[kC];
#pragma unroll
    for (int q = 0; q < kC; ++q) {
        const int r = 4 * (wv * kC + q) + (lane >> 4);
        const int c = (lane & 15) ^ pf_swz(r);
        off[q] = static_cast<int64_t>(min(key0 + r, k_last)) * row_bytes + 16 * c;
    }
#pragma unroll
    for (int q = 0; q < kC; ++q)
        __builtin_amdgcn_global_load_lds(seg + off[q], (lds_void_t*)(dst + (wv * kC + q) * 1024), 16, 0, kNt);
}

// Running state of a piece in lane (g, n): O^T[16dt + 4g + i][column n] in fp64, the
// lane's share of the column's sum, and the column's running max (log2 units, integer-
// valued; -inf until the piece has seen a key the column may attend to).  V^T P^T of the
// windows since the last kMtGroup boundary is summed in fp32 (acc) and then moved into the
// fp64 O: fp32 sums over 128 keys add no error measurable against per-window sums, and
// the move costs two VALU instructions per element.
constexpr int kMtGroup = 4;
struct MtState {
    double o64[8][4];
    f32x4_t acc[8];
    double l64;
    float m_run;
    int grp;                  // windows summed into acc
};

__device__ __forceinline__ void mt_flush(MtState& t) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) t.o64[dt][i] += static_cast<double>(t.acc[dt][i]);
        t.acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    t.grp = 0;
}

// The cached keys' statistics of a piece for the rescore flag (the largest squared norm of
// each K pair group and the largest |V| of each dim over the piece's keys below the chunk),
// kept per lane until the piece ends and formed without branches (a branch between an MFMA
// and the read of its result can lose the wait states the read needs).
//  * One tile (W = 1, one wave per SIMD, registers to spare): from the operands the wave
//    already holds.  K: lane (g, n) reads key 16 kt + n, dims 32 kb + 8g .. +7 in slice kb,
//    so slices kb and kb + 2 together hold pair group 4 (kb & 1) + g whole: kmax[kb & 1].
//    V: the V^T operand of dim tile dt gives lane (g, n) 8 keys of dim 16 dt + n: vmax[dt].
//  * Two or four tiles (their registers are all in use): each wave reads its 32/W keys of
//    the window from LDS, K beside the window's scores, V after its V^T P^T.  K: lane l
//    takes key (l >> 3) (+ 8 j) and the two 16-byte chunks of pair group l & 7: kmax[0].
//    V: lane l takes dims 8 (l & 15) .. +7 of key (l >> 4) (+ 4 j): vmax[0..3].
template <int kW>
struct MtStats {
    static constexpr int kNk = kW == 1 ? 2 : 1;
    static constexpr int kNv = kW == 1 ? 8 : 4;
    uint32_t kmax[kNk];                             // squared group norms, fp32 bits
    uint32_t vmax[kNv];                             // two |V| codes per dword
};

template <int kW>
__device__ __forceinline__ void mt_stats_reset(MtStats<kW>& ms) {
#pragma unroll
    for (int i = 0; i < MtStats<kW>::kNk; ++i) ms.kmax[i] = 0u;
#pragma unroll
    for (int i = 0; i < MtStats<kW>::kNv; ++i) ms.vmax[i] = 0u;
}

// The stages of one 32-key window [key0, key0 + 32) of a piece ending at k_b, for this
// wave's tile.  mt_qk: the raw scores S^T = K Q^T of both 16-key tiles from the K plane, and
// the squared pair-group norms of the window's first klim keys (the cached keys of the piece;
// none when klim <= 0): one tile from its operands, two or four from this wave's share of
// the plane.
template <int kW>
__device__ __forceinline__ void mt_qk(const uint8_t* kplane, const bf16x8_t (&qop)[3][4], int wv, int lane,
                                      f32x4_t (&sacc)[2], int klim, MtStats<kW>& ms) {
    const int n = lane & 15;
    const int g = lane >> 4;
    sacc[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    sacc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float nrm[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        bf16x8_t ak[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) ak[kt] = pf_k_chunk(kplane, 16 * kt + n, 4 * kb + g);
#pragma unroll
        for (int s = 0; s < 3; ++s)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[kt], qop[s][kb], sacc[kt], 0, 0, 0);
        if constexpr (kW == 1) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const uint4 w = __builtin_bit_cast(uint4, ak[kt]);
                nrm[kt][kb & 1] =
                    bf16x2_sq_acc(w.w, bf16x2_sq_acc(w.z, bf16x2_sq_acc(w.y, bf16x2_sq_acc(w.x, nrm[kt][kb & 1]))));
            }
        }
    }
    if constexpr (kW == 1) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                const uint32_t x = 16 * kt + n < klim ? __float_as_uint(nrm[kt][pr]) : 0u;
                ms.kmax[pr] = max(ms.kmax[pr], x);
            }
    } else {
        mt_stats_k<kW>(kplane, wv, lane, klim, ms);
    }
}

// The |V| code masks of one tile's V^T operand dwords (element 2j + h of lane (g, n)'s 8 is
// key 16 (j / 2) + 4g + 2 (j % 2) + h): the first vlim keys of the window count.
__device__ __forceinline__ void mt_vmask(int vlim, int lane, uint32_t (&vm)[4]) {
    const int g = lane >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k0 = 16 * (j >> 1) + 4 * g + 2 * (j & 1);
        vm[j] = (k0 < vlim ? 0x7fffu : 0u) | (k0 + 1 < vlim ? 0x7fff0000u : 0u);
    }
}

// Two or four tiles: this wave's share of a window's statistics from its planes in LDS
// (keys (32 / W) wv + ..), the first lim keys of the window counting.  K is taken from the
// plane the window's scores are formed from (one window ahead: the ring refills a K slot with
// a later V before the next barrier, so a K plane is not read once its window is current);
// V from the current window's plane.
template <int kW>
__device__ __forceinline__ void mt_stats_k(const uint8_t* kplane, int wv, int lane, int lim, MtStats<kW>& ms) {
    constexpr int kKeys = kMtWin / kW;
    const int c = lane & 7;
#pragma unroll
    for (int j = 0; j < kKeys / 8; ++j) {
        const int row = kKeys * wv + 8 * j + (lane >> 3);
        const uint4 lo = __builtin_bit_cast(uint4, pf_k_chunk(kplane, row, c));
        const uint4 hi = __builtin_bit_cast(uint4, pf_k_chunk(kplane, row, c + 8));
        float sq = bf16x2_sq_acc(lo.x, 0.f);
        sq = bf16x2_sq_acc(lo.y, sq);
        sq = bf16x2_sq_acc(lo.z, sq);
        sq = bf16x2_sq_acc(lo.w, sq);
        sq = bf16x2_sq_acc(hi.x, sq);
        sq = bf16x2_sq_acc(hi.y, sq);
        sq = bf16x2_sq_acc(hi.z, sq);
        sq = bf16x2_sq_acc(hi.w, sq);
        ms.kmax[0] = max(ms.kmax[0], row < lim ? __float_as_uint(sq) : 0u);
    }
}

// V: lane l takes dims 8 (l & 15) .. +7 of key (l >> 4) (+ 4 j): one 16-byte read per lane
// and four keys per instruction; the lanes of a dim are combined once per piece.
template <int kW>
__device__ __forceinline__ void mt_stats_v(const uint8_t* vplane, int wv, int lane, int lim, MtStats<kW>& ms) {
    constexpr int kKeys = kMtWin / kW;
    const int vc = lane & 15;
#pragma unroll
    for (int j = 0; j < kKeys / 4; ++j) {
        const int row = kKeys * wv + 4 * j + (lane >> 4);
        const uint4 x = __builtin_bit_cast(uint4, pf_k_chunk(vplane, row, vc));
        const uint32_t m = row < lim ? 0x7fff7fffu : 0u;
        ms.vmax[0] = pk_max_u16(ms.vmax[0], x.x & m);
        ms.vmax[1] = pk_max_u16(ms.vmax[1], x.y & m);
        ms.vmax[2] = pk_max_u16(ms.vmax[2], x.z & m);
        ms.vmax[3] = pk_max_u16(ms.vmax[3], x.w & m);
    }
}

// mt_max: chunk keys (>= st) take the scores the preparation formed from their unrounded
// rows (`cs`: this lane's column against chunk keys u = 0 .. kU-1); keys past the piece or
// past the column's token (`lim` = start + t) are masked; the window max per column updates
// the running max (rescaling O and l by an exact power of two).  Returns the max the
// probabilities are taken against.
template <int kU>
__device__ __forceinline__ float mt_max(const PrefillArgs& a, bool chunk_keys, const float (&cs)[kU], int st,
                                        int key0, int k_b, int lim, int lane, f32x4_t (&sacc)[2], MtState& t) {
    const int g = lane >> 4;
    if (chunk_keys) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int u = key0 + 16 * kt + 4 * g + i - st;
                if (u >= 0 && u < a.n_new) {
                    // cs[u] by bit masks (a select chain is turned into an indexed load from
                    // a stack copy; masking keeps a NaN in another entry out of this one).
                    uint32_t vb = 0u;
#pragma unroll
                    for (int q = 0; q < kU; ++q) vb |= __float_as_uint(cs[q]) & (u == q ? 0xFFFFFFFFu : 0u);
                    sacc[kt][i] = __uint_as_float(vb);
                }
            }
    }
    // Masks: only a window holding chunk keys (the causal limit lim >= start) or running past
    // the piece has any (a uniform test).
    if (chunk_keys || key0 + kMtWin > k_b) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = key0 + 16 * kt + 4 * g + i;
                if (key >= k_b || key > lim) sacc[kt][i] = -INFINITY;
            }
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) bmax = fmaxf(bmax, sacc[kt][i]);
    bmax = swap32_max(swap16_max(bmax));
    const float m_new = bmax > t.m_run ? ceilf(bmax) : t.m_run;
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
        t.m_run = m_new;
    }
    // A column that has seen no key yet keeps m = -inf and p = 0 (every score -inf).
    return t.m_run == -INFINITY ? 0.f : t.m_run;
}

// mt_probs: p = 2^(s - m) in three BF16 parts (the P^T B operand), summed into l.
__device__ __forceinline__ void mt_probs(const f32x4_t (&sacc)[2], float m_eff, uint32_t (&ph)[3][2][4], MtState& t) {
    float lsum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) pf_probs_tile(sacc[kt], m_eff, lsum, ph, kt);
    t.l64 += static_cast<double>(lsum);
}

// mt_pv: O^T += V^T P^T of this window (its V in LDS, visible to every wave): dim tile dt
// from two transposed reads (rows 4g + a/4 and 16 rows on), summed in fp32 into the group's
// acc, which every kMtGroup windows moves into the fp64 O (the caller's mt_flush).
template <int kW>
__device__ __forceinline__ void mt_pv(uint32_t vbase, const uint32_t (&ph)[3][2][4], int lane, MtState& t,
                                      const uint32_t (&vm)[4], MtStats<kW>& ms) {
    bf16x8_t pb[3];
#pragma unroll
    for (int s = 0; s < 3; ++s) pb[s] = as_bf16x8(make_uint4(ph[s][0][0], ph[s][0][1], ph[s][0][2], ph[s][0][3]));
#pragma unroll
    for (int d0 = 0; d0 < 8; d0 += 2) {
        // Inline reads: the compiler does not see them as LDS accesses, so it adds no wait for
        // the window copies in flight (the reads' own wait is explicit).
        short4_t r[2][2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t ad = vbase + vt_tr_offset(d0 + e, lane);
            asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r[e][0]) : "v"(ad));
            asm volatile("ds_read_b64_tr_b16 %0, %1 offset:4096" : "=v"(r[e][1]) : "v"(ad));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0][0]), "+v"(r[0][1]), "+v"(r[1][0]), "+v"(r[1][1]));
        bf16x8_t av[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            union {
                short4_t h[2];
                bf16x8_t v;
            } u;
            u.h[0] = r[e][0];
            u.h[1] = r[e][1];
            av[e] = u.v;
            if constexpr (kW == 1) {
                // The |V| codes of the window's cached keys (masks from mt_vmask).
                const uint4 w = __builtin_bit_cast(uint4, u.v);
                uint32_t& m = ms.vmax[d0 + e];
                m = pk_max_u16(m, pk_max_u16(pk_max_u16(w.x & vm[0], w.y & vm[1]), pk_max_u16(w.z & vm[2], w.w & vm[3])));
            }
        }
#pragma unroll
        for (int s = 0; s < 3; ++s)
#pragma unroll
            for (int e = 0; e < 2; ++e)
                t.acc[d0 + e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[e], pb[s], t.acc[d0 + e], 0, 0, 0);
    }
    ++t.grp;
}

// End of a piece: the column sums over the four rows; a whole segment writes its output
// rows (tokens < T), a split one its partial at slot wg + segment, columns 16 wv + n, in
// fp32: its rounding (2^-24 of the partial, about 6e-8 of an output row's rms) is far below
// the kernel's own error, and a row with an element near zero, where it could matter, is
// flagged by the merge and rescored in fp64.
template <int kW>
__device__ __forceinline__ void mt_piece_end(const PrefillArgs& a, int b, int kvh, bool whole, int64_t slot,
                                             int wv, int lane, MtState& t) {
    const int n = lane & 15;
    const int g = lane >> 4;
    const double l = swap_add_f64<true>(swap_add_f64<false>(t.l64));
    if (whole) {
        const int tok = 4 * wv + (n >> 2);
        // Column n's row (lanes n, n+16, n+32, n+48 hold dims 16dt + 4g ..).
        double x[8][4];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[dt][i] = t.o64[dt][i] / l;
        if (tok >= a.n_new) return;
        if (g == 0 && a.rs_hdr)
            a.rs_m[(static_cast<int64_t>(b) * a.n_new + tok) * kHq + kvh * kGroup + (n & 3)] = t.m_run;
        uint16_t* orow = a.out + ((static_cast<int64_t>(b) * a.n_new + tok) * kHq + kvh * kGroup + (n & 3)) * kD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            uint2 pk;
            pk.x = f32_to_bf16_out(static_cast<float>(x[dt][0])) |
                   (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(x[dt][1]))) << 16);
            pk.y = f32_to_bf16_out(static_cast<float>(x[dt][2])) |
                   (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(x[dt][3]))) << 16);
            *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * g) = pk;
        }
        return;
    }
    const int64_t col = slot * (kMtTile * kW) + kMtTile * wv + n;
    float* po = a.part_o + col * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<float4*>(po + 16 * dt + 4 * g) =
            make_float4(static_cast<float>(t.o64[dt][0]), static_cast<float>(t.o64[dt][1]),
                        static_cast<float>(t.o64[dt][2]), static_cast<float>(t.o64[dt][3]));
    if (g == 0) a.part_ml[col] = make_float2(t.m_run, static_cast<float>(l));
}

// End of a piece's statistics: each value reduced over the lanes that hold it, then stored
// into the piece's slot (wg + segment, as its partial), one record per wave; the merge kernel
// reduces a segment's records into its maxima.  Plain stores, one writer per
// record (atomic maxima from every piece onto a segment's 136 words instead: B=64 ragged
// T = 8 and 16 stream kernels 2-3 us slower).
template <int kW>
__device__ __forceinline__ void mt_stats_end(const PrefillArgs& a, int64_t slot, int wv, int lane, MtStats<kW>& ms) {
    uint32_t* kdst = a.piece_st + (slot * kW + wv) * (8 + kD);
    uint32_t* ddst = kdst + 8;
    if constexpr (kW == 1) {
        const int n = lane & 15;
        const int g = lane >> 4;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint32_t x = ms.kmax[i];
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) x = max(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), sh)));
            if (n == 0) kdst[4 * i + g] = x;
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            uint32_t x = ms.vmax[dt];
            x = pk_max_u16(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), 16)));
            x = pk_max_u16(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), 32)));
            x = max(x & 0xffffu, x >> 16);
            if (g == 0) ddst[16 * dt + n] = x;
        }
    } else {
        uint32_t x = ms.kmax[0];
#pragma unroll
        for (int sh = 8; sh < kWave; sh <<= 1) x = max(x, static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), sh)));
        if (lane < 8) kdst[lane] = x;
        uint32_t* dc = ddst + 8 * (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t v = ms.vmax[i];
            v = pk_max_u16(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 16)));
            v = pk_max_u16(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 32)));
            if (lane < 16) {
                dc[2 * i] = v & 0xffffu;
                dc[2 * i + 1] = v >> 16;
            }
        }
    }
    mt_stats_reset<kW>(ms);
}

// Sequence windows of the plan: o = seq_off[base + lane], o1 = seq_off[base + lane + 1].
struct MtWindow {
    int base;
    int64_t o, o1;
};

__device__ __forceinline__ void mt_load_window(const PrefillArgs& a, int base, MtWindow& w) {
    const int bb = base + static_cast<int>(threadIdx.x & (kWave - 1));
    w.base = base;
    w.o = bb < a.batch ? a.seq_off[bb] : INT64_MAX;
    w.o1 = bb < a.batch ? a.seq_off[bb + 1] : INT64_MAX;
}

// The segment after (b, kvh) that has keys; false when there is none.
__device__ __forceinline__ bool mt_next_segment(const PrefillArgs& a, MtWindow& w, int lead, int& b, int& kvh,
                                                int& nk) {
    if (kvh + 1 < kHkv) {
        ++kvh;
        return true;
    }
    kvh = 0;
    while (true) {
        const int bb = w.base + static_cast<int>(threadIdx.x & (kWave - 1));
        const uint64_t m = __ballot(bb < a.batch && bb > b && w.o1 > w.o);
        if (m) {
            const int j = __ffsll(static_cast<unsigned long long>(m)) - 1;
            b = w.base + j;
            nk = static_cast<int>((__shfl(w.o1, j) - __shfl(w.o, j)) / kHkv) - lead;
            return true;
        }
        if (w.base + kWave >= a.batch) return false;
        mt_load_window(a, w.base + kWave, w);
    }
}

// A position in a workgroup's window stream: piece keys [pk, k_b) of segment (b, kvh)
// (nk keys), current window at key kw, x = stream position of key pk; `sw` is the plan's
// sequence window around b.  mt_advance moves to the next window of the piece, else to the
// first window of the next piece, else marks the cursor invalid.
struct MtCursor {
    int b, kvh, nk, pk, k_b, kw;
    int64_t x;
    int64_t seg_elem;         // element offset of segment (b, kvh) in the cache, formed once
                              // per segment (not per copy: B=64 T=16 274.5 -> 270.3 us)
    bool valid;
    MtWindow sw;
};

__device__ __forceinline__ void mt_advance(const PrefillArgs& a, MtCursor& c, int64_t x_end, int lead) {
    if (c.kw + kMtWin < c.k_b) {
        c.kw += kMtWin;
        return;
    }
    const int64_t x_next = c.x + (c.k_b - c.pk);
    int b = c.b, kvh = c.kvh, nk = c.nk;
    bool more = x_next + lead < x_end;
    if (more) more = mt_next_segment(a, c.sw, lead, b, kvh, nk);
    if (!more) {
        c.valid = false;
        return;
    }
    c.b = __builtin_amdgcn_readfirstlane(b);
    c.kvh = __builtin_amdgcn_readfirstlane(kvh);
    c.nk = __builtin_amdgcn_readfirstlane(nk);
    c.seg_elem = static_cast<int64_t>(c.b) * a.kv_batch_stride + static_cast<int64_t>(c.kvh) * a.kv_head_stride;
    c.x = uniform_i64(x_next + lead);
    c.pk = 0;
    c.kw = 0;
    c.k_b = __builtin_amdgcn_readfirstlane(static_cast<int>(min(static_cast<int64_t>(c.nk), x_end - c.x)));
}

// Eight f32 values split into three BF16 parts each, packed as three MFMA operands (two
// values per dword): hi = x truncated to 8 significant bits, mid = the residual truncated,
// lo = what remains, which has at most 8 significant bits -- every step exact, so
// hi + mid + lo = x.
__device__ __forceinline__ void mt_split3_8(const float (&x)[8], uint4 (&w)[3]) {
    float r1[8], r2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        r1[i] = x[i] - __uint_as_float(__float_as_uint(x[i]) & 0xffff0000u);
        r2[i] = r1[i] - __uint_as_float(__float_as_uint(r1[i]) & 0xffff0000u);
    }
    w[0] = make_uint4(pack_hi16(x[0], x[1]), pack_hi16(x[2], x[3]), pack_hi16(x[4], x[5]), pack_hi16(x[6], x[7]));
    w[1] = make_uint4(pack_hi16(r1[0], r1[1]), pack_hi16(r1[2], r1[3]), pack_hi16(r1[4], r1[5]), pack_hi16(r1[6], r1[7]));
    w[2] = make_uint4(pack_hi16(r2[0], r2[1]), pack_hi16(r2[2], r2[3]), pack_hi16(r2[4], r2[5]), pack_hi16(r2[6], r2[7]));
}

template <int kW>
// Two- and four-tile workgroups run two waves per SIMD: their registers (VGPRs and AGPRs
// together) must fit in half the SIMD's file.
__global__ __launch_bounds__(kWave * kW) __attribute__((amdgpu_waves_per_eu(kW == 1 ? 1 : 2))) void mt_stream_kernel(PrefillArgs a) {
    constexpr int kA = mt_ahead(kW);
    constexpr int kS = mt_slots(kW);
    constexpr int kC = kMtCopies / kW;
    constexpr int kU = 4 * kW;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kS * kMtPlaneB];
    MtWindow w0;
    mt_load_window(a, 0, w0);
    const int64_t wg = blockIdx.x;
    const int64_t total = a.plan_hdr[0];
    const int64_t per_wg = a.plan_hdr[1];
    const int lead = static_cast<int>(a.plan_hdr[2]);
    const int64_t extra = a.plan_hdr[3];
    int64_t x = range_start(per_wg, extra, wg);
    if (x >= total) return;
    const int64_t x_end = min(range_start(per_wg, extra, wg + 1), total);
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & (kWave - 1);
    const int n = lane & 15;
    const int64_t row_bytes = a.kv_pos_stride * 2;
    const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(lds)));

    // First piece: the last sequence b with seq_off[b] <= x.
    MtCursor c;
    int64_t off = 0, next = 0;
    c.b = 0;
    for (int base = 0; base < a.batch; base += kWave) {
        MtWindow t = w0;
        if (base > 0) mt_load_window(a, base, t);
        const uint64_t le = __ballot(t.o <= x);
        if (le) {
            const int j = 63 - __clzll(static_cast<long long>(le));
            c.b = base + j;
            off = __shfl(t.o, j);
            next = __shfl(t.o1, j);
            c.sw = t;
        }
    }
    int kvh, key, nk;
    locate_first_piece(off, next, lead, x, kvh, key, nk);
    c.x = uniform_i64(x);
    c.b = __builtin_amdgcn_readfirstlane(c.b);
    c.kvh = __builtin_amdgcn_readfirstlane(kvh);
    c.seg_elem = static_cast<int64_t>(c.b) * a.kv_batch_stride + static_cast<int64_t>(c.kvh) * a.kv_head_stride;
    c.pk = __builtin_amdgcn_readfirstlane(key);
    c.kw = c.pk;
    c.nk = __builtin_amdgcn_readfirstlane(nk);
    c.k_b = __builtin_amdgcn_readfirstlane(static_cast<int>(min(static_cast<int64_t>(c.nk), c.pk + (x_end - c.x))));
    c.valid = true;

    auto slot_ptr = [&](int sl) { return lds + (sl >= kS ? sl - kS : sl) * kMtPlaneB; };
    auto issue = [&](const uint16_t* base, const MtCursor& q, int sl) {
        mt_issue_plane<kC>(reinterpret_cast<const char*>(base + q.seg_elem), row_bytes, q.kw, q.k_b - 1, slot_ptr(sl), wv, lane);
    };
    // The producer p is the last window whose K copies were requested; the consumer c's
    // window has K in slot `slot` and V in the next one.  kq = windows after c's whose K
    // has been requested (at most kA before the window's own requests).
    MtCursor p = c;
    int slot = 0, kq = 0;
    issue(a.k, p, 0);
#pragma unroll
    for (int j = 0; j < kA; ++j) {
        if (p.valid) {
            issue(a.v, p, 2 * j + 1);
            mt_advance(a, p, x_end, lead);
            if (p.valid) {
                issue(a.k, p, 2 * j + 2);
                ++kq;
            }
        }
    }

    MtStats<kW> ms;
    mt_stats_reset<kW>(ms);
    while (true) {
        // This piece: Q operands, chunk-key scores, start, window loop.
        const int st = a.start[c.b];
        const int64_t seg = static_cast<int64_t>(c.b) * kHkv + c.kvh;
        bf16x8_t qop[3][4];
        {
            const float4* src = a.q_op + (seg * kW + wv) * 8 * kWave + lane;
            float4 qf[8];
#pragma unroll
            for (int f = 0; f < 8; ++f) qf[f] = src[f * kWave];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const float x[8] = {qf[2 * kb].x, qf[2 * kb].y, qf[2 * kb].z, qf[2 * kb].w,
                                    qf[2 * kb + 1].x, qf[2 * kb + 1].y, qf[2 * kb + 1].z, qf[2 * kb + 1].w};
                uint4 w[3];
                mt_split3_8(x, w);
#pragma unroll
                for (int sp = 0; sp < 3; ++sp) qop[sp][kb] = as_bf16x8(w[sp]);
            }
        }
        float cs[kU];
        {
            const float4* src = reinterpret_cast<const float4*>(a.chunk_s + (seg * (kMtTile * kW) + kMtTile * wv + n) * kU);
#pragma unroll
            for (int q = 0; q < kW; ++q) {
                const float4 v = src[q];
                cs[4 * q] = v.x;
                cs[4 * q + 1] = v.y;
                cs[4 * q + 2] = v.z;
                cs[4 * q + 3] = v.w;
            }
        }
        const int lim = st + min(4 * wv + (n >> 2), a.n_new - 1);
        MtState t;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) t.o64[dt][i] = 0.0;
            t.acc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        t.l64 = 0.0;
        t.m_run = -INFINITY;
        t.grp = 0;

        // Each window's scores are formed one window ahead, their MFMAs beside the current
        // window's probabilities (the next window's K plane is in LDS: K runs kA + 1 windows
        // ahead).  B=64 ragged: T=8 302.4 -> 287.9 us per step, T=4 216.2 -> 215.2.  The
        // piece's first window's scores are formed here (its V(i + kA) not yet requested).
        f32x4_t s_cur[2];
        mt_wait_planes<kC, 2 * kA>(kq == kA);
        mt_barrier();
        // Keys of the piece below the chunk: the ones its statistics cover.
        const int stat_end = min(c.k_b, st);
        mt_qk<kW>(slot_ptr(slot), qop, wv, lane, s_cur, stat_end - c.kw, ms);
        for (;;) {
            // Request V of the producer's window (kA after this one) and, once every wave
            // is done with the previous window, K of the window after it.
            const bool iv = p.valid;
            if (iv) issue(a.v, p, slot + 2 * kA + 1);
            const bool has_next = c.kw + kMtWin < c.k_b;
            if (has_next) mt_wait_planes<kC, 2 * kA - 1>(kq == kA);   // K of the next window landed
            mt_barrier();
            bool ik = false;
            if (iv) {
                mt_advance(a, p, x_end, lead);
                if (p.valid) {
                    issue(a.k, p, slot + 2 * kA + 2);
                    ik = true;
                }
            }
            const bool v_steady = kq == kA && ik;     // 2 kA + 1 planes requested after V
            const bool chunk_keys = c.kw + kMtWin > st;
            // A piece's last window waited for no next K: wait for its V and meet here.
            // Otherwise the wait above covered it: every wave requested this window's V
            // before the next window's K, and the copies complete in issue order (B=64
            // ragged, T=16: stream kernel 283 -> 272 us).
            if (!has_next) {
                mt_wait_planes<kC, 2 * kA + 1>(v_steady);
                mt_barrier();
            }
            if (t.grp == kMtGroup) mt_flush(t);
            uint32_t ph[3][2][4];
            const float m_eff = mt_max(a, chunk_keys, cs, st, c.kw, c.k_b, lim, lane, s_cur, t);
            // One branch-free block: the next window's scores (on a piece's last window the
            // plane read is the next piece's or stale, and the result is dropped), this
            // window's probabilities, V^T P^T and statistics.
            f32x4_t s_next[2];
            mt_qk<kW>(slot_ptr(slot + 2), qop, wv, lane, s_next, stat_end - (c.kw + kMtWin), ms);
            mt_probs(s_cur, m_eff, ph, t);
            uint32_t vm[4] = {0u, 0u, 0u, 0u};
            if constexpr (kW == 1) mt_vmask(stat_end - c.kw, lane, vm);
            mt_pv<kW>(lds_base + (slot + 1 >= kS ? slot + 1 - kS : slot + 1) * kMtPlaneB, ph, lane, t, vm, ms);
            if constexpr (kW > 1)
                mt_stats_v<kW>(slot_ptr(slot + 1), wv, lane, stat_end - c.kw, ms);
            s_cur[0] = s_next[0];
            s_cur[1] = s_next[1];
            slot = slot + 2 >= kS ? slot + 2 - kS : slot + 2;
            kq = ik ? kq : kq - 1;
            if (!has_next) break;
            c.kw += kMtWin;
        }
        mt_flush(t);
        mt_piece_end<kW>(a, c.b, c.kvh, c.pk == 0 && c.k_b == c.nk, wg + seg, wv, lane, t);
        mt_stats_end<kW>(a, wg + seg, wv, lane, ms);
        mt_advance(a, c, x_end, lead);
        if (!c.valid) break;
    }
}

// The rescore flag of one output row, where the row is final: lane j of the row's 16 lanes
// holds dims 8j .. 8j+7 (BF16 codes ow), which lie in pair group j % 8.  The keys token t
// sees: its segment's cached keys (their maxima seg_st: the 8 pair-group norms, then the
// |V| code of each dim) and the chunk's rows up to its own (rs_kpre / rs_dpre, the running
// maxima the preparation left).  The elements in units of their dim's largest |V| (a dim
// whose V is zero in every key the row sees is exactly zero and left out) and the scores'
// bound E = scale log2(e) sum_G |q_G| max|k_G| decide (rs_flag_decide); Q's pair-group norms
// come from the row as given, which rotation leaves unchanged.  y and its square are formed
// in double: y is at most 1 in magnitude (an output element is a weighted mean of its dim's
// V) but may be far smaller -- keys of huge V that the softmax gives no weight set D_j and not
// the output -- and in fp32 y^2 underflows to zero in every dim once the row's elements lie
// ~2^63 below their D_j, which leaves nothing to compare (BF16 ratios lie within 2^+-261 and
// their squares within double's range).  E stays in fp32: it only overflows to infinity
// (the row is then rescored) or underflows to zero (F = 1 then, the N(0,1) threshold).
// What the decision reads from memory, loaded before the merge so that it is in flight
// beside the partials: this lane's 8 Q values, the chunk rows' |V| maxima at its dims and
// the pair-group norm maximum of its group.
struct MtFlagIn {
    uint4 qx, dp;
    uint32_t kpre;
};

__device__ __forceinline__ void mt_flag_load(const PrefillArgs& a, int64_t bh, int t, int64_t row, int j,
                                             MtFlagIn& in) {
    const int64_t er = bh * a.n_new + t;
    in.qx = *reinterpret_cast<const uint4*>(a.q + row * kD + 8 * j);
    in.dp = *reinterpret_cast<const uint4*>(a.rs_dpre + er * kD + 8 * j);
    in.kpre = a.rs_kpre[er * 8 + (j & 7)];
}

__device__ __forceinline__ void mt_flag_row(const PrefillArgs& a, int64_t row, float m, const uint32_t (&ow)[4],
                                            const MtFlagIn& in, const uint32_t* seg_st, int j) {
    const uint4 qx = in.qx, dp = in.dp;
    const uint32_t kq = max(seg_st[j & 7], in.kpre);
    const uint32_t dw[4] = {dp.x, dp.y, dp.z, dp.w};
    const uint32_t qw[4] = {qx.x, qx.y, qx.z, qx.w};
    double ss = 0.0, mn2 = INFINITY;
    float qq = 0.f;
    bool bad = false, vinf = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t d = max(seg_st[8 + 8 * j + i], i & 1 ? dw[i >> 1] >> 16 : dw[i >> 1] & 0xffffu);
        const uint32_t xs = i & 1 ? ow[i >> 1] & 0xffff0000u : ow[i >> 1] << 16;
        const uint32_t qs = i & 1 ? qw[i >> 1] & 0xffff0000u : qw[i >> 1] << 16;
        const float x = __uint_as_float(xs), q = __uint_as_float(qs);
        const float dv = __uint_as_float(d << 16);
        const double y = dv > 0.f ? static_cast<double>(x) * __builtin_amdgcn_rcp(static_cast<double>(dv)) : 0.0;
        ss = fma(y, y, ss);
        if (dv > 0.f) mn2 = fmin(mn2, y * y);
        bad |= !__builtin_isfinite(x);
        vinf |= !(dv <= 3.4028235e38f);             // an infinite or NaN V among the row's keys
        qq = fmaf(q, q, qq);
    }
    // |q_G| |k_G|max: lanes j and j + 8 hold the two halves of pair group j % 8.
    qq += dpp_f<0x128>(qq);                         // row_ror:8
    float e = j < 8 ? sqrtf(qq) * sqrtf(__uint_as_float(kq)) : 0.f;
    ss = row16_sum_f64(ss);
    e = row16_sum(e);
    mn2 = row16_min_f64(mn2);
    const uint64_t bads = __ballot(bad);
    const int h = (threadIdx.x & (kWave - 1)) >> 4;
    const bool row_bad = ((bads >> (16 * h)) & 0xffffull) != 0ull;
    const bool row_vinf = ((__ballot(vinf) >> (16 * h)) & 0xffffull) != 0ull;
    // A key whose p falls below fp32's normal range is lost to v_exp_f32's flush or to the
    // BF16 split, at most ~2^-124 of weight each (p <= 1 against the running max, the ceiling
    // of the largest score, so l >= 1/2).  Harmless unless its V is near the BF16 maximum,
    // where it can outweigh the output: every element is within capacity * 2^-123 of its D_j,
    // and a row with an element below 8 times that (|y_j| < capacity * 2^-120) is rescored too.
    const double tq = static_cast<double>(a.capacity) * 0x1p-120;
    if (j == 0 && (row_bad || mn2 < tq * tq ||
                   rs_flag_decide(mn2, ss, static_cast<double>(m), static_cast<double>(e) * fabs(a.qk_scale_log2)))) {
        rs_append(a, static_cast<uint32_t>(row));
        if (row_vinf) atomicOr(a.rs_hdr + 2, 1u);
    }
}

// One workgroup per (KV head, sequence), 16 threads per column: thread i handles column
// i/16 (token c/4, head c%4), dims 8(i%16) .. +8.  It reduces the segment's cached-key
// maxima from every piece's records, merges the partials of a split segment's pieces
// (weights 2^(m - max) are exact; a piece that saw no key the column may attend to has
// m = -inf and weight 0) and decides each output row's rescore flag.
template <int kW>
__global__ __launch_bounds__(256 * kW) __attribute__((amdgpu_waves_per_eu(8))) void mt_merge_kernel(PrefillArgs a) {
    constexpr int kCols = kMtTile * kW;
    const int kvh = blockIdx.x;
    const int b = blockIdx.y;
    const int64_t per_wg = a.plan_hdr[1];
    const int lead = static_cast<int>(a.plan_hdr[2]);
    const int64_t extra = a.plan_hdr[3];
    const int64_t off = a.seq_off[b];
    const int span = static_cast<int>((a.seq_off[b + 1] - off) / kHkv);
    if (span == 0) return;                          // no keys: a start out of range, NaN rows
    const int nk = span - lead;
    const int64_t seg_off = off + static_cast<int64_t>(kvh) * span + lead;
    const int64_t w_first = range_of(per_wg, extra, seg_off);
    const int n_pieces = static_cast<int>(range_of(per_wg, extra, seg_off + nk - 1) - w_first) + 1;
    const int64_t slot0 = w_first + static_cast<int64_t>(b) * kHkv + kvh;
    const int64_t bh = static_cast<int64_t>(b) * kHkv + kvh;
    const int col = threadIdx.x >> 4;
    const int j = threadIdx.x & 15;
    const int d0 = 8 * j;
    const int tok = col >> 2;
    const bool live = tok < a.n_new;
    const int64_t row = (static_cast<int64_t>(b) * a.n_new + min(tok, a.n_new - 1)) * kHq + kvh * kGroup + (col & 3);
    // The flag's inputs (and a whole segment's row, which the stream kernel wrote with its
    // running max) requested first.
    MtFlagIn fin{};
    uint32_t ow[4] = {0u, 0u, 0u, 0u};
    float m = 0.f;
    if (a.rs_hdr && live) {
        mt_flag_load(a, bh, tok, row, j, fin);
        if (n_pieces == 1) {
            const uint2* src = reinterpret_cast<const uint2*>(a.out + row * kD + d0);   // out is 8-byte aligned
            const uint2 x0 = src[0], x1 = src[1];
            ow[0] = x0.x;
            ow[1] = x0.y;
            ow[2] = x1.x;
            ow[3] = x1.y;
            m = a.rs_m[row];
        }
    }
    __shared__ uint32_t seg_st[8 + kD];
    if (a.rs_hdr && threadIdx.x < 8 + kD) {
        // Four pieces' records at a time, all requested before any is used.
        uint32_t x = 0u;
        for (int p0 = 0; p0 < n_pieces; p0 += 4) {
            uint32_t r[4][kW];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int w = 0; w < kW; ++w)
                    r[q][w] = p0 + q < n_pieces ? a.piece_st[((slot0 + p0 + q) * kW + w) * (8 + kD) + threadIdx.x] : 0u;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int w = 0; w < kW; ++w) x = max(x, r[q][w]);
        }
        seg_st[threadIdx.x] = x;
    }
    mt_lds_barrier();
    if (!live) return;
    if (n_pieces > 1) {
        // Pieces two at a time, every load of a group issued before any is used (one memory
        // round trip per group; with 61 registers eight waves fit on a SIMD, so a 16-wave
        // workgroup per segment at T = 16 no longer leaves half of them waiting for a CU);
        // the running max moves by whole powers of two, so rescaling what is already summed
        // is exact.
        constexpr int kGroupP = 2;
        m = -INFINITY;
        double l = 0.0, o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int p0 = 0; p0 < n_pieces; p0 += kGroupP) {
            float2 ml[kGroupP];
            float v[kGroupP][8];                        // widened where summed
#pragma unroll
            for (int q = 0; q < kGroupP; ++q) {
                ml[q] = make_float2(-INFINITY, 0.f);
                if (p0 + q < n_pieces) {
                    const int64_t c = (slot0 + p0 + q) * kCols + col;
                    ml[q] = a.part_ml[c];
                    const float4* po = reinterpret_cast<const float4*>(a.part_o + c * kD + d0);
                    const float4 x0 = po[0], x1 = po[1];
                    v[q][0] = x0.x;
                    v[q][1] = x0.y;
                    v[q][2] = x0.z;
                    v[q][3] = x0.w;
                    v[q][4] = x1.x;
                    v[q][5] = x1.y;
                    v[q][6] = x1.z;
                    v[q][7] = x1.w;
                }
            }
            float mb = m;
#pragma unroll
            for (int q = 0; q < kGroupP; ++q) mb = fmaxf(mb, ml[q].x);
            if (m != -INFINITY && mb != m) {
                const int e = max_shift(m, mb);
                l = ldexp(l, e);
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = ldexp(o[i], e);
            }
            m = mb;
#pragma unroll
            for (int q = 0; q < kGroupP; ++q) {
                if (ml[q].x == -INFINITY) continue;
                const int e = max_shift(ml[q].x, m);
                l += ldexp(static_cast<double>(ml[q].y), e);
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] += ldexp(static_cast<double>(v[q][i]), e);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ow[i] = f32_to_bf16_out(static_cast<float>(o[2 * i] / l)) |
                    (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(o[2 * i + 1] / l))) << 16);
        uint2* dst = reinterpret_cast<uint2*>(a.out + row * kD + d0);   // out is 8-byte aligned
        dst[0] = make_uint2(ow[0], ow[1]);
        dst[1] = make_uint2(ow[2], ow[3]);
    }
    if (a.rs_hdr) mt_flag_row(a, row, m, ow, fin, seg_st, j);
}

template <int kW>
hipError_t launch_multi_w(const PrefillArgs& a, hipStream_t stream, hipEvent_t* ev) {
    const bool vec = (reinterpret_cast<uintptr_t>(a.q) % 16) == 0 && (reinterpret_cast<uintptr_t>(a.k_new) % 16) == 0;
    const dim3 grid(kHkv, static_cast<unsigned>(a.batch) + 1);
    // A failed launch still records the events this function owns (1 .. kProfileEvents - 2),
    // so that the profiler can read the call's stage times.
    auto done = [&](int from, hipError_t err) {
        if (ev)
            for (int j = from; j < kProfileEvents - 1; ++j) (void)hipEventRecord(ev[j], stream);
        return err;
    };
    if (vec)
        hipLaunchKernelGGL((mt_prepare_kernel<true, kW>), grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((mt_prepare_kernel<false, kW>), grid, dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return done(1, e);
    if (ev) (void)hipEventRecord(ev[1], stream);
    hipLaunchKernelGGL(mt_stream_kernel<kW>, dim3(static_cast<unsigned>(a.n_wgs)), dim3(kWave * kW), 0, stream, a);
    e = hipGetLastError();
    if (ev) (void)hipEventRecord(ev[2], stream);
    if (e != hipSuccess) return done(3, e);
    hipLaunchKernelGGL(mt_merge_kernel<kW>, dim3(kHkv, static_cast<unsigned>(a.batch)), dim3(256 * kW), 0, stream, a);
    e = hipGetLastError();
    if (ev) (void)hipEventRecord(ev[3], stream);
    return e;
}

hipError_t launch_prefill_multi(const PrefillArgs& a, hipStream_t stream, hipEvent_t* ev) {
    if (multi_waves(a.n_new) == 1) return launch_multi_w<1>(a, stream, ev);
    if (multi_waves(a.n_new) == 2) return launch_multi_w<2>(a, stream, ev);
    return launch_multi_w<4>(a, stream, ev);
}

}  // namespace gqa

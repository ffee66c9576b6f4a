// gqa_decode.hip -- GQA decode for gfx950: one persistent launch, stream-K split over
// all keys of the batch, QK^T on MFMA, weighted V on fp64 VALU, exact merge of pieces.
//
// One decode step of the reference core (gqa_controller.v:140-277 loop nest, datapath
// rope_unit -> bf16_dot_product_mac -> scale_unit -> flash_softmax ->
// output_accumulator -> gqa_output_collector) is decode_stream_kernel, a persistent
// grid of n_wgs one-wave workgroups:
//
//  * The keys of every (sequence, kv_head) segment are laid end to end (segment =
//    b*8 + h, n_valid(b) keys each) and cut into n_wgs equal ranges, one per
//    workgroup, so every wave streams the same number of K/V rows whatever the
//    length mix.  The part of one segment inside one range is a "piece".
//  * Inside a piece the wave rotates and scales the 4 Q rows of its group once and
//    reuses every K/V row for the 4 Q heads (gqa_kv_broadcast.v:38-59), keeping the
//    next 16-key chunk in flight while it computes the current one.
//  * A piece that is a whole segment normalises and writes its 4 output rows
//    (output_accumulator.v:540-686, BF16 in Q-head order, gqa_output_collector.v:32-61).
//    Otherwise it leaves an unnormalised partial (O[4][128] fp64, running max m,
//    sum l) at slot wg + segment -- unique because both increase along the key
//    order -- and bumps the segment's counter; the piece that finishes last merges
//    all partials of the segment and resets the counter for the next call.
//
// Arithmetic (the golden model is double, pyfiles/gen_gqa_wrapper_vectors.py:121-139):
//  * Q is rotated in double, scaled by scale*log2(e) in double and split into three
//    BF16 parts (hi, mid, lo: ~26 significant bits).  K is BF16 already, so the
//    bf16 x bf16 MFMA products are exact and the scores carry fp32 accumulation
//    error only.  With RoPE on K (the reference's unrotated cache) the rotated K row
//    is split the same way.
//  * The running max m is kept integer-valued (m = ceil(max score)), so every
//    rescale of the accumulator and every combine weight is an exact power of two.
//  * p = exp2(s - m) in fp32; the weighted-V accumulation and the combine run in
//    fp64 (full-rate on CDNA4), so their rounding never reaches the BF16 output.
//
// Masking (gqa_attention_wrapper.v:279): key p counts iff p < seq_len and
// p <= query_position.  Only keys p < n_valid = min(seq_len, qpos+1) are ever
// loaded; inside the last chunk the other lanes load nothing, score -inf and get
// p = 0 exactly (flash_softmax.v:319-325).
//
// Lane layouts (wave64, l = lane):
//  * QK, MFMA f32_16x16x32_bf16 with A = K (row = key l%16), B = Q^T (column
//    n = l%16: n = 4*split + head for n < 12, zero for n >= 12).  Lane group
//    g = l/16 and element j of MFMA kb cover head dim d = 32*kb + 8*g + j, so a
//    lane loads 16 contiguous bytes per kb and holds both halves (d, d+64) of its
//    RoPE pairs (kb and kb+2).  Output lane l holds score(key 4g+i, column n).
//  * PV: lane (r = l/16, c = l%16) owns dims [8c, 8c+8) of key 4*it + r of the
//    chunk; one 16-byte load per lane covers four whole V rows (1 KB contiguous).
#include "gqa_device.h"
#include "gqa_internal.h"

namespace gqa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunk = 16;           // keys per MFMA group
constexpr int kMinRangeKeys = 64;    // smallest per-workgroup key range

__device__ __forceinline__ int seq_valid_keys(const DecodeArgs& a, int b) {
    const int L = a.seq_len[b];
    const int qp = a.query_pos[b];
    if (L < 1 || L > a.capacity || qp < 0 || qp >= L) return 0;
    return min(L, qp + 1);
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t x) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) x += __shfl_xor(x, d);
    return x;
}

__device__ __forceinline__ int64_t wave_incl_scan_i64(int64_t x, int lane) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int64_t y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

// Total keys over all segments (8 per sequence) and the per-workgroup range size.
__device__ __forceinline__ void stream_totals(const DecodeArgs& a, int lane, int64_t& total,
                                              int64_t& per_wg) {
    int64_t t = 0;
    for (int base = 0; base < a.batch; base += kWave) {
        const int b = base + lane;
        t += wave_sum_i64(b < a.batch ? seq_valid_keys(a, b) : 0);
    }
    total = t * kHkv;
    int64_t per = (total + a.n_wgs - 1) / a.n_wgs;
    per = per < kMinRangeKeys ? kMinRangeKeys : per;
    per_wg = (per + kChunk - 1) / kChunk * kChunk;
}

// Sequence whose segments contain global key offset x (0 <= x < total):
// returns b and off_b = 8 * (valid keys of sequences before b).
__device__ __forceinline__ int locate_sequence(const DecodeArgs& a, int lane, int64_t x,
                                               int64_t& off_b) {
    int64_t carry = 0;
    for (int base = 0; base < a.batch; base += kWave) {
        const int b = base + lane;
        const int64_t nv = b < a.batch ? seq_valid_keys(a, b) : 0;
        const int64_t incl = wave_incl_scan_i64(nv, lane) + carry;
        const uint64_t past = __ballot((incl * kHkv) > x);
        if (past) {
            const int first = __ffsll(static_cast<unsigned long long>(past)) - 1;
            off_b = (__shfl(incl, first) - __shfl(nv, first)) * kHkv;
            return base + first;
        }
        carry = __shfl(incl, kWave - 1);
    }
    off_b = carry * kHkv;
    return a.batch;   // unreachable for x < total
}

// BF16 code of a double, rounding through f32 (any nearby BF16 value serves as the
// leading part of a split; the residual is formed exactly in double).
__device__ __forceinline__ uint16_t bf16_of(double d) { return f32_to_bf16_rne(static_cast<float>(d)); }

__device__ __forceinline__ double f64_of_bf16(uint16_t b) { return static_cast<double>(bf16_to_f32(b)); }

// Split v into hi + mid + lo BF16 codes; returns part `which`.
__device__ __forceinline__ uint16_t split3(double v, int which) {
    const uint16_t hi = bf16_of(v);
    const double r1 = v - f64_of_bf16(hi);
    const uint16_t mid = bf16_of(r1);
    if (which == 0) return hi;
    if (which == 1) return mid;
    return bf16_of(r1 - f64_of_bf16(mid));
}

__device__ __forceinline__ bf16x8_t pack8(const uint16_t (&h)[8]) {
    union {
        uint16_t u[8];
        bf16x8_t v;
    } t;
#pragma unroll
    for (int j = 0; j < 8; ++j) t.u[j] = h[j];
    return t.v;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& w) {
    union {
        uint4 u;
        bf16x8_t v;
    } t;
    t.u = w;
    return t.v;
}

// K and V rows of one 16-key chunk, in the MFMA (K) and PV (V) lane layouts.
struct Chunk {
    uint4 kw[4];
    uint4 vw[4];
};

// Running state of one piece: fp64 weighted-V accumulator (4 heads x this lane's 8 dims),
// integer-valued running max and partial sum (head n in lanes n < 4).
struct PieceState {
    double acc[kGroup][8];
    float m_run;
    float l_run;
};

__device__ __forceinline__ void load_chunk(const uint16_t* kbase, const uint16_t* vbase,
                                           int64_t ps, int kc, int k_b, int n, int g, Chunk& c) {
    const int kkey = kc + n;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        c.kw[kb] = make_uint4(0, 0, 0, 0);
        if (kkey < k_b) c.kw[kb] = *reinterpret_cast<const uint4*>(kbase + kkey * ps + 32 * kb);
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int vkey = kc + 4 * it + g;
        c.vw[it] = make_uint4(0, 0, 0, 0);
        if (vkey < k_b) c.vw[it] = *reinterpret_cast<const uint4*>(vbase + vkey * ps);
    }
}

// Scores, online softmax and weighted V of one chunk [kc, kc+16) (keys >= k_b masked).
template <bool kRopeK>
__device__ __forceinline__ void compute_chunk(const DecodeArgs& a, int kc, int k_b, int n, int g,
                                              const Chunk& c, const bf16x8_t (&bq)[4],
                                              PieceState& st, float (*p_tile)[kGroup]) {
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
    if (kRopeK) {
        // Rotate the K row at its position: pairs (kb, kb+2) of this lane.
        const int kkey = kc + n;
        double kr[4][8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            float xf[8], yf[8];
            unpack8(c.kw[kb], xf);
            unpack8(c.kw[kb + 2], yf);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                double xr, yr;
                rope_pair(xf[j], yf[j], kkey, a.rope.inv_freq[32 * kb + 8 * g + j], xr, yr);
                kr[kb][j] = xr;
                kr[kb + 2][j] = yr;
            }
        }
#pragma unroll
        for (int part = 0; part < 3; ++part) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                uint16_t h8[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) h8[j] = split3(kr[kb][j], part);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pack8(h8), bq[kb], d, 0, 0, 0);
            }
        }
    } else {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(c.kw[kb]), bq[kb], d, 0, 0, 0);
    }
    // Sum the hi/mid/lo columns n, n+4, n+8 into every lane of the same n%4 (columns
    // 12..15 are zero, so the rotations by 4, 8 and 12 within the 16-lane row add exactly those).
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x = d[i];
        s[i] = x + dpp_f<0x124>(x) + dpp_f<0x128>(x) + dpp_f<0x12C>(x);
        if (kc + 4 * g + i >= k_b) s[i] = -INFINITY;
    }

    // Online softmax (head n in lanes n < 4; m integer-valued so rescales are exact).
    float cm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    cm = fmaxf(cm, __shfl_xor(cm, 16));
    cm = fmaxf(cm, __shfl_xor(cm, 32));
    const bool grow = (n < kGroup) && (cm > st.m_run);
    if (__ballot(grow)) {
        const float m_new = grow ? ceilf(cm) : st.m_run;
        // 2^(m_run - m_new), exact; 0 when nothing has been accumulated yet.
        const int shift = (st.m_run == -INFINITY) ? -1100 : static_cast<int>(st.m_run - m_new);
        st.l_run = ldexpf(st.l_run, max(shift, -200));
        st.m_run = m_new;
        int sh[kGroup];
#pragma unroll
        for (int h = 0; h < kGroup; ++h) sh[h] = __shfl(shift, h);
#pragma unroll
        for (int h = 0; h < kGroup; ++h) {
            if (sh[h] != 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) st.acc[h][j] = ldexp(st.acc[h][j], sh[h]);
            }
        }
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[i] = (s[i] == -INFINITY) ? 0.f : exp2f(s[i] - st.m_run);
        st.l_run += p[i];
    }
    if (n < kGroup) {
#pragma unroll
        for (int i = 0; i < 4; ++i) p_tile[4 * g + i][n] = p[i];
    }
    __syncthreads();

    // Weighted V in fp64.
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const float4 p4 = *reinterpret_cast<const float4*>(&p_tile[4 * it + g][0]);
        float vf[8];
        unpack8(c.vw[it], vf);
        double vd[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vd[j] = static_cast<double>(vf[j]);
        const double pd[kGroup] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
        for (int h = 0; h < kGroup; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) st.acc[h][j] = fma(pd[h], vd[j], st.acc[h][j]);
    }
}

// Merge the pieces of segment (b, kvh) -- slots w + seg for w in [w_first, w_last] --
// with exact power-of-two weights in fp64; write the 4 output rows.  Lane: 2 dims.
__device__ __forceinline__ void combine_segment(const DecodeArgs& a, int b, int kvh, int64_t seg,
                                                int64_t w_first, int64_t w_last) {
    const int lane = threadIdx.x;
#pragma unroll 1
    for (int h = 0; h < kGroup; ++h) {
        float mx = -INFINITY;
        for (int64_t w = w_first; w <= w_last; ++w)
            mx = fmaxf(mx, a.part_ml[(w + seg) * kGroup + h].x);
        double l = 0.0, o0 = 0.0, o1 = 0.0;
        for (int64_t w = w_first; w <= w_last; ++w) {
            const int64_t slot = w + seg;
            const float2 ml = a.part_ml[slot * kGroup + h];
            const int e = max(static_cast<int>(ml.x - mx), -1100);
            const double2 o = reinterpret_cast<const double2*>(a.part_o + (slot * kGroup + h) * kD)[lane];
            l += ldexp(static_cast<double>(ml.y), e);
            o0 += ldexp(o.x, e);
            o1 += ldexp(o.y, e);
        }
        uint32_t* out = reinterpret_cast<uint32_t*>(
            a.out + (static_cast<int64_t>(b) * kHq + kvh * kGroup + h) * kD);
        const uint32_t lo = f32_to_bf16_rne(static_cast<float>(o0 / l));
        const uint32_t hi = f32_to_bf16_rne(static_cast<float>(o1 / l));
        out[lane] = lo | (hi << 16);
    }
}

// One piece: keys [k_a, k_b) of segment (b, kvh), which starts at global key offset
// seg_off.  Writes the output rows itself when the piece is the whole segment;
// otherwise leaves a partial, and the last piece of the segment to finish merges all.
template <bool kRopeQ, bool kRopeK>
__device__ __forceinline__ void process_piece(const DecodeArgs& a, int b, int kvh, int nv, int k_a,
                                              int k_b, int64_t seg_off, int64_t per_wg,
                                              int64_t wg, double (*q_s)[kD],
                                              float (*p_s)[kChunk][kGroup]) {
    const int lane = threadIdx.x;
    const int n = lane & 15;       // MFMA column / PV dim chunk
    const int g = lane >> 4;       // MFMA lane group / PV key row
    const int qpos = a.query_pos[b];

    const int64_t head_off = static_cast<int64_t>(b) * a.kv_batch_stride +
                             static_cast<int64_t>(kvh) * a.kv_head_stride;
    const int64_t ps = a.kv_pos_stride;
    const uint16_t* kbase = a.k + head_off + 8 * g;        // + key*ps + 32*kb
    const uint16_t* vbase = a.v + head_off + 8 * n;        // + key*ps

    // First chunk's rows are requested before the Q prologue so that their latency
    // overlaps it.
    Chunk c0, c1;
    load_chunk(kbase, vbase, ps, k_a, k_b, n, g, c0);

    // ---- Q rows of the group: rotate at qpos and scale, in double.
    __syncthreads();
    {
        double sn = 0.0, cs = 1.0;
        if (kRopeQ) sincos(static_cast<double>(qpos) * a.rope.inv_freq[lane], &sn, &cs);
#pragma unroll
        for (int h = 0; h < kGroup; ++h) {
            const uint16_t* qrow = a.q + (static_cast<int64_t>(b) * kHq + kvh * kGroup + h) * kD;
            const double x = bf16_to_f32(qrow[lane]);
            const double y = bf16_to_f32(qrow[lane + kPairs]);
            double xr = x, yr = y;
            if (kRopeQ) {
                xr = x * cs - y * sn;
                yr = x * sn + y * cs;
            }
            q_s[h][lane] = xr * a.qk_scale_log2;
            q_s[h][lane + kPairs] = yr * a.qk_scale_log2;
        }
    }
    __syncthreads();
    // MFMA B operand: column n -> split n/4 of head n%4 (zero for n >= 12).
    bf16x8_t bq[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        uint16_t h8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            h8[j] = n < 12 ? split3(q_s[n & 3][32 * kb + 8 * g + j], n >> 2) : uint16_t(0);
        bq[kb] = pack8(h8);
    }

    PieceState st;
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) st.acc[h][j] = 0.0;
    st.m_run = -INFINITY;
    st.l_run = 0.f;

    // Two register sets: chunk j+1 is in flight while chunk j is computed.
    for (int kc = k_a;; kc += 2 * kChunk) {
        const bool more1 = kc + kChunk < k_b;
        if (more1) load_chunk(kbase, vbase, ps, kc + kChunk, k_b, n, g, c1);
        compute_chunk<kRopeK>(a, kc, k_b, n, g, c0, bq, st, p_s[0]);
        if (!more1) break;
        const bool more2 = kc + 2 * kChunk < k_b;
        if (more2) load_chunk(kbase, vbase, ps, kc + 2 * kChunk, k_b, n, g, c0);
        compute_chunk<kRopeK>(a, kc + kChunk, k_b, n, g, c1, bq, st, p_s[1]);
        if (!more2) break;
    }

    // ---- sum the four key rows; every lane then holds the totals.
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            st.acc[h][j] += __shfl_xor(st.acc[h][j], 16);
            st.acc[h][j] += __shfl_xor(st.acc[h][j], 32);
        }
    st.l_run += __shfl_xor(st.l_run, 16);
    st.l_run += __shfl_xor(st.l_run, 32);

    const int64_t seg = static_cast<int64_t>(b) * kHkv + kvh;
    if (k_a == 0 && k_b == nv) {
        // The whole segment: normalise in fp64, round double -> f32 -> BF16.
        double lh[kGroup];
#pragma unroll
        for (int h = 0; h < kGroup; ++h) lh[h] = static_cast<double>(__shfl(st.l_run, h));
        if (g == 0) {
#pragma unroll
            for (int h = 0; h < kGroup; ++h) {
                uint16_t o8[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) o8[j] = f32_to_bf16_rne(static_cast<float>(st.acc[h][j] / lh[h]));
                uint4 pk;
                pk.x = o8[0] | (static_cast<uint32_t>(o8[1]) << 16);
                pk.y = o8[2] | (static_cast<uint32_t>(o8[3]) << 16);
                pk.z = o8[4] | (static_cast<uint32_t>(o8[5]) << 16);
                pk.w = o8[6] | (static_cast<uint32_t>(o8[7]) << 16);
                *reinterpret_cast<uint4*>(a.out + (static_cast<int64_t>(b) * kHq + kvh * kGroup + h) * kD +
                                          8 * n) = pk;
            }
        }
        return;
    }

    const int64_t slot = wg + seg;
    if (g == 0) {
#pragma unroll
        for (int h = 0; h < kGroup; ++h) {
            double2* dst = reinterpret_cast<double2*>(a.part_o + (slot * kGroup + h) * kD + 8 * n);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j] = make_double2(st.acc[h][2 * j], st.acc[h][2 * j + 1]);
        }
    }
    if (lane < kGroup) a.part_ml[slot * kGroup + lane] = make_float2(st.m_run, st.l_run);

    // Count finished pieces; the last one merges.  Release the partial before the
    // count, acquire the others' after it (device scope: the pieces ran on other CUs
    // and XCDs).
    __threadfence();
    int done = 0;
    if (lane == 0) done = atomicAdd(&a.counters[seg], 1);
    done = __shfl(done, 0);
    const int64_t w_first = seg_off / per_wg;
    const int64_t w_last = (seg_off + nv - 1) / per_wg;
    if (done == static_cast<int>(w_last - w_first)) {
        __threadfence();
        combine_segment(a, b, kvh, seg, w_first, w_last);
        if (lane == 0) atomicExch(&a.counters[seg], 0);   // ready for the next call
    }
}

template <bool kRopeQ, bool kRopeK>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(2))) void decode_stream_kernel(DecodeArgs a) {
    __shared__ double q_s[kGroup][kD];
    __shared__ float p_s[2][kChunk][kGroup];
    const int lane = threadIdx.x;
    const int64_t w = blockIdx.x;

    // Sequences whose lengths break the rules get NaN rows (and no reads):
    // workgroup w checks sequences w, w + n_wgs, ...
    for (int64_t bb = w; bb < a.batch; bb += a.n_wgs) {
        if (seq_valid_keys(a, static_cast<int>(bb)) == 0) {
            uint4* out = reinterpret_cast<uint4*>(a.out + bb * kHq * kD);
            for (int i = lane; i < kHq * kD / 8; i += kWave)
                out[i] = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
        }
    }

    int64_t total, per_wg;
    stream_totals(a, lane, total, per_wg);
    int64_t x = w * per_wg;
    if (x >= total) return;
    const int64_t x_end = min(x + per_wg, total);

    int64_t off_b;
    int b = locate_sequence(a, lane, x, off_b);
    int nvb = seq_valid_keys(a, b);
    int kvh = static_cast<int>((x - off_b) / nvb);
    int key = static_cast<int>((x - off_b) % nvb);
    while (true) {
        const int k_b = static_cast<int>(min(static_cast<int64_t>(nvb), key + (x_end - x)));
        process_piece<kRopeQ, kRopeK>(a, b, kvh, nvb, key, k_b, x - key, per_wg, w, q_s, p_s);
        x += k_b - key;
        if (x >= x_end) break;
        key = 0;
        if (++kvh == kHkv) {
            kvh = 0;
            nvb = 0;
            while (nvb == 0 && ++b < a.batch) nvb = seq_valid_keys(a, b);
            if (nvb == 0) break;   // lengths changed under the launch; nothing left to read
        }
    }
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

hipError_t launch_zero_words(uint32_t* p, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(zero_words_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       stream, p, n);
    return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, int batch, hipStream_t stream, hipEvent_t* ev) {
    const dim3 grid_stream(a.n_wgs);
    const bool rq = (a.flags & 1u) != 0, rk = (a.flags & 2u) != 0;
    if (ev) (void)hipEventRecord(ev[0], stream);
    if (rq && rk)
        hipLaunchKernelGGL((decode_stream_kernel<true, true>), grid_stream, dim3(kWave), 0, stream, a);
    else if (rq)
        hipLaunchKernelGGL((decode_stream_kernel<true, false>), grid_stream, dim3(kWave), 0, stream, a);
    else if (rk)
        hipLaunchKernelGGL((decode_stream_kernel<false, true>), grid_stream, dim3(kWave), 0, stream, a);
    else
        hipLaunchKernelGGL((decode_stream_kernel<false, false>), grid_stream, dim3(kWave), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ev) {
        (void)hipEventRecord(ev[1], stream);
        (void)hipEventRecord(ev[2], stream);
    }
    (void)batch;
    return e;
}

}  // namespace gqa

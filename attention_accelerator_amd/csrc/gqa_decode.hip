// gqa_decode.hip -- GQA decode for gfx950: a persistent stream-K split over all keys
// of the batch, scores and weighted V on fp64 MFMA, exact merge of pieces.
//
// One decode step of the reference core (gqa_controller.v:140-277 loop nest, datapath
// rope_unit -> bf16_dot_product_mac -> scale_unit -> flash_softmax ->
// output_accumulator -> gqa_output_collector) is, by default, three launches on one
// stream: decode_prepare_kernel (the plan of pieces below, and every segment's 4 Q rows
// rotated and scaled once), decode_stream_kernel (a persistent grid of n_wgs one-wave
// workgroups) and decode_merge_kernel:
//
//  * The keys of every (sequence, kv_head) segment are laid end to end (segment =
//    b*8 + h, n_valid(b) keys each; in a batch of segments shorter than a few ranges,
//    each preceded by a lead of positions that stands for a piece's fixed cost) and cut
//    into n_wgs equal ranges, one per workgroup, so every wave takes about as long
//    whatever the length mix.  The part of one segment's keys inside one range is a
//    "piece".
//  * Inside a piece the wave reuses every K/V row for the 4 Q heads of its group
//    (gqa_kv_broadcast.v:38-59), keeping the next 16-key chunk in flight while it
//    computes the current one; the next piece's first chunk is requested before the
//    current piece ends.
//  * A piece that is a whole segment normalises and writes its 4 output rows
//    (output_accumulator.v:540-686, BF16 in Q-head order, gqa_output_collector.v:32-61).
//    Otherwise it leaves an unnormalised partial (O[4][128] fp64, running max m,
//    sum l) at slot wg + segment -- unique because both increase along the key
//    order -- and decode_merge_kernel, launched next on the same stream, merges the
//    pieces of each such segment; the kernel boundary orders the partials.
//
// Other launch shapes of the same step: decode_single_kernel (small batches: one launch,
// one 4-wave workgroup per piece of a segment, the last piece of a segment to finish
// merges it after an agent-scope counter) and decode_paged_stream_kernel (the stream
// kernel over a block-table cache).
//
// Arithmetic (the golden model is double, pyfiles/gen_gqa_wrapper_vectors.py:121-139):
// every step is carried in fp64, so the output differs from the golden's double value by
// double roundings only, far below one BF16 ULP of any output that is not exactly zero.
//  * Q is rotated at query_position in double and scaled by scale*log2(e) in double.
//  * Scores: fp64 MFMA (v_mfma_f64_4x4x4_4b_f64) of the K values (BF16, exact in double;
//    with RoPE on K the row is rotated in double first) and the fp64 Q.
//  * The running max m is kept integer-valued in double (m = ceil(max score)), so every
//    rescale of the accumulator and every combine weight is an exact power of two, also
//    for scores past 2^24, where an fp32 m could not stay within a few units of them.
//  * p = exp2(s - m) in fp64; weighted V by fp64 MFMA; l, the merge and the division in
//    fp64; the row is rounded double -> f32 -> BF16 as the reference's f32_to_bf16.
//
// Masking (gqa_attention_wrapper.v:279): key p counts iff p < seq_len and
// p <= query_position.  Only keys p < n_valid = min(seq_len, qpos+1) are ever
// loaded; inside the last chunk the other lanes load a clamped row, score -inf and get
// p = 0 exactly (flash_softmax.v:319-325).
//
// Lane layouts of one 16-key chunk (wave64, l = lane).  v_mfma_f64_4x4x4_4b_f64 runs four
// 4x4x4 blocks; lane l holds A[m = l%4][k = l/16] and B[k = l/16][n = l%4] of block
// (l/4)%4 and receives C[m = l/16][n = l%4] of that block.
//  * QK^T: A = K (block row = key l%16), B = Q^T (column = head l%4); MFMA (kb, e), kb,
//    e < 4, 8, takes head dim 32kb + 8(l/16) + e in k-slot l/16, so a lane loads 16
//    contiguous bytes of its key's row per kb and holds both halves (d, d+64) of its RoPE
//    pairs (kb and kb+2).  C: lane l holds the score of key 4((l/4)%4) + l/16, head l%4.
//  * PV: A = V^T, B = P: MFMA (q, e) takes keys 4q + k in k-slot k, and block b's rows
//    m are dims 8(4b + m) + e, so V load q of lane l is 16 contiguous bytes of row
//    4q + l/16, dims 8(l%16) .. -- four whole rows per load instruction.  B lane l holds
//    p of head l%4, key 4q + l/16, gathered through 512 bytes of LDS from the score lanes.
//    C: lane l accumulates O[head l%4][8(4((l/4)%4) + l/16) + e] over all keys.
#include "gqa_device.h"
#include "gqa_internal.h"
#include "gqa_streamk.h"

namespace gqa {

constexpr int kChunk = 16;           // keys per MFMA group

__device__ __forceinline__ int seq_valid_keys(const DecodeArgs& a, int b) {
    const int L = a.seq_len[b];
    const int qp = a.query_pos[b];
    if (L < 1 || L > a.capacity || qp < 0 || qp >= L) return 0;
    return min(L, qp + 1);
}

// Keys of sequence b's segments in the stream-K key space: n_valid, rounded up to the
// 16-position block for a paged cache so that every piece starts on a block.
__device__ __forceinline__ int plan_keys(const DecodeArgs& a, int b) {
    const int nv = seq_valid_keys(a, b);
    return a.block_table ? (nv + kChunk - 1) / kChunk * kChunk : nv;
}

// Span of each of sequence b's segments in the stream (gqa_streamk.h).
__device__ __forceinline__ int plan_span(const DecodeArgs& a, int b, int lead) {
    const int k = plan_keys(a, b);
    return k > 0 ? k + lead : 0;
}

// Stream positions over all segments (8 per sequence), the per-workgroup range size and
// the segment lead.
__device__ __forceinline__ void stream_totals(const DecodeArgs& a, int lane, int64_t& total, int64_t& per_wg,
                                              int& lead) {
    int64_t sum = 0;
    int max_keys = 0, n_seq = 0;
    for (int base = 0; base < a.batch; base += kWave) {
        const int b = base + lane;
        const int k = b < a.batch ? plan_keys(a, b) : 0;
        sum += wave_sum_i64(k);
        max_keys = max(max_keys, static_cast<int>(wave_max_i64(k)));
        n_seq += static_cast<int>(wave_sum_i64(k > 0 ? 1 : 0));
    }
    plan_lead_totals(sum, max_keys, n_seq, a.n_wgs, lead, total, per_wg);
}

// Key of lane l's score within a chunk (the QK^T output layout).
__device__ __forceinline__ int chunk_key_of_lane(int lane) { return 4 * ((lane >> 2) & 3) + (lane >> 4); }

// First of the 8 output dims lane l accumulates (PV output layout), head l%4.
__device__ __forceinline__ int out_dim_of_lane(int lane) { return 8 * (4 * ((lane >> 2) & 3) + (lane >> 4)); }

// K and V rows of one 16-key chunk: kw[kb] = 8 K values of key l%16, dims 32kb + 8(l/16)..;
// vw[q] = 8 V values of key 4q + l/16, dims 8(l%16)...
struct Chunk {
    uint4 kw[4];
    uint4 vw[4];
};

// Running state of one piece in lane l: O[head l%4][out_dim_of_lane(l) + e] in acc[e], and
// the head's integer-valued running max (double, as every step here: scores may lie far
// beyond 2^24) and (this lane's share of the) sum of p.  m_run is the same in every lane
// of a head.
struct PieceState {
    double acc[8];
    double l_run;
    double m_run;
};

__device__ __forceinline__ void init_piece(PieceState& st) {
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = 0.0;
    st.l_run = 0.0;
    st.m_run = -INFINITY;
}

// The 32 Q values lane l feeds the QK^T MFMAs: q[kb][e] = Q[head l%4][32kb + 8(l/16) + e],
// rotated and scaled by scale*log2(e) in double.
struct QOps {
    double q[4][8];
};

// Byte offsets (from the segment's first K / V row) of this lane's rows in the current
// chunk.  Loads are unconditional so that the compiler counts them exactly (a load
// under a branch makes it wait for every outstanding load at the join, prefetches
// included); rows past the piece are clamped to its last row and masked afterwards.
struct ChunkRows {
    uint32_t k;       // key kc + l%16, + 16*(l/16) bytes into the row
    uint32_t v[4];    // key kc + 4q + l/16, + 16*(l%16) bytes into the row
};

__device__ __forceinline__ void load_chunk(const char* kseg, const char* vseg, const ChunkRows& r,
                                           uint32_t k_last, uint32_t v_last, Chunk& c) {
    const char* kp = kseg + min(r.k, k_last);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) c.kw[kb] = load_stream16(kp + 64 * kb);
#pragma unroll
    for (int q = 0; q < 4; ++q) c.vw[q] = load_stream16(vseg + min(r.v[q], v_last));
}

__device__ __forceinline__ void advance(ChunkRows& r, uint32_t step) {
    r.k += step;
#pragma unroll
    for (int q = 0; q < 4; ++q) r.v[q] += step;
}

__device__ __forceinline__ double mfma_f64(double a, double b, double c) {
    return __builtin_amdgcn_mfma_f64_4x4x4f64(a, b, c, 0, 0, 0);
}

// Scores may exceed the running reference m by this much (log2 units) before it is raised:
// p <= 2^64 and a piece's l <= 2^95 (still an fp32 in the partial record).
constexpr double kMaxHeadroom = 64.0;

// 2^x for finite x <= kMaxHeadroom + 1, relative error below 1e-14: x = n + f with
// n = rint(x), |f| <= 1/2, and 2^f = e^t, t = f ln 2, by its Taylor series to degree 11
// (truncation error < (ln2/2)^12 / 12! < 7e-15).  x below about -1075 gives 0.
__device__ __forceinline__ double exp2_f64(double x) {
    const double n = rint(x);
    const double t = (x - n) * 0.6931471805599453094;
    double y = 1.0 / 39916800.0;              // 1/11!
    y = fma(y, t, 1.0 / 3628800.0);           // 1/10!
    y = fma(y, t, 1.0 / 362880.0);
    y = fma(y, t, 1.0 / 40320.0);
    y = fma(y, t, 1.0 / 5040.0);
    y = fma(y, t, 1.0 / 720.0);
    y = fma(y, t, 1.0 / 120.0);
    y = fma(y, t, 1.0 / 24.0);
    y = fma(y, t, 1.0 / 6.0);
    y = fma(y, t, 0.5);
    y = fma(y, t, 1.0);
    y = fma(y, t, 1.0);
    return ldexp(y, static_cast<int>(fmax(n, -2000.0)));
}

// Scores, online softmax and weighted V of one chunk [kc, kc+16) (keys >= k_b masked).
// kRope: each K row is rotated first, at position rope_pos0 + its key index.
template <int kRope>
__device__ __forceinline__ void compute_chunk(const RopeTable& rope, int rope_pos0, int kc, int k_b, const Chunk& c,
                                              const QOps& qa, PieceState& st) {
    // p exchange slice of this wave (workgroups of up to four waves).
    __shared__ double p_lds[4][kWave];
    double* pl = p_lds[(threadIdx.x >> 6) & 3];
    const int lane = threadIdx.x & (kWave - 1);
    // QK^T: four independent accumulation chains (one per kb), summed in a fixed order.
    double s4[4] = {0.0, 0.0, 0.0, 0.0};
    if (kRope) {
        // Rotate the K row at its position in double: pairs (kb, kb+2) of this lane.
        const int kkey = kc + (lane & 15);
        const int g = lane >> 4;
        double kr[4][8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            float xf[8], yf[8];
            unpack8(c.kw[kb], xf);
            unpack8(c.kw[kb + 2], yf);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int fi = 32 * kb + 8 * g + j;
                double xr, yr;
                rope_pair(xf[j], yf[j], rope_pos0 + kkey, rope.inv_freq[fi], xr, yr);
                kr[kb][j] = xr;
                kr[kb + 2][j] = yr;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) s4[kb] = mfma_f64(kr[kb][e], qa.q[kb][e], s4[kb]);
    } else {
        // Every K value converted first, then the 32 MFMAs back to back: VALU work does not
        // overlap an fp64 MFMA on gfx950, and interleaving adds wait states between them.
        double kd[4][8];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            float kf[8];
            unpack8(c.kw[kb], kf);
#pragma unroll
            for (int e = 0; e < 8; ++e) kd[kb][e] = static_cast<double>(kf[e]);
        }
        __builtin_amdgcn_sched_group_barrier(0x002, 64, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) s4[kb] = mfma_f64(kd[kb][e], qa.q[kb][e], s4[kb]);
    }
    const int key = kc + chunk_key_of_lane(lane);
    double s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    if (key >= k_b) s = -INFINITY;

    // Online softmax per head with a lazy reference: m (integer-valued, common to the 16
    // lanes with lane%4 == head) is raised only when a score exceeds m + kMaxHeadroom, so
    // the rescale below runs about once per piece; p = 2^(s - m) <= 2^kMaxHeadroom then,
    // far inside the fp64 range.  The new m is the ceiling of the head's chunk max over its
    // 16 lanes (rows through lane swaps, blocks through row rotations).
    if (__ballot(s > st.m_run + kMaxHeadroom)) {
        double cm = s;
        cm = fmax(cm, dpp_d<0x124>(cm));
        cm = fmax(cm, dpp_d<0x128>(cm));
        cm = swap_max_f64<true>(swap_max_f64<false>(cm));
        const bool grow = cm > st.m_run + kMaxHeadroom;
        const double m_new = grow ? ceil(cm) : st.m_run;
        // 2^(m_run - m_new), exact; nothing has been accumulated while m_run is -inf.
        const int shift = (st.m_run == -INFINITY) ? 0 : max_shift_f64(st.m_run, m_new);
        st.l_run = ldexp(st.l_run, shift);
#pragma unroll
        for (int i = 0; i < 8; ++i) st.acc[i] = ldexp(st.acc[i], shift);
        st.m_run = m_new;
    }
    // p = 0 for a masked key (and for every key while m is -inf, when all of them are).  The
    // clamp keeps a NaN (a NaN score, or +inf against a running max raised to +inf): as in
    // the golden's exp(s - max), it makes the row NaN (fmax would turn it into p = 0).
    const double xs = s - st.m_run;
    const double p = key < k_b ? exp2_f64(xs < -2000.0 ? -2000.0 : xs) : 0.0;
    st.l_run += p;

    // p of (head l%4, key 4q + l/16) for q = 0..3, from the lane holding that score
    // (lane 16(key%4) + 4(key/4) + head): through LDS, [row l/16][head][q].
    pl[(lane >> 4) * 16 + (lane & 3) * 4 + ((lane >> 2) & 3)] = p;
    const double2 pa = *reinterpret_cast<const double2*>(pl + (lane >> 4) * 16 + (lane & 3) * 4);
    const double2 pb = *reinterpret_cast<const double2*>(pl + (lane >> 4) * 16 + (lane & 3) * 4 + 2);
    const double pq[4] = {pa.x, pa.y, pb.x, pb.y};

    // Weighted V.  A masked key's V row is a clamped row of the piece, weighted by p = 0.
    double vd[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float vf[8];
        unpack8(c.vw[q], vf);
#pragma unroll
        for (int e = 0; e < 8; ++e) vd[q][e] = static_cast<double>(vf[e]);
    }
    if (kc + kChunk > k_b) {
        // A chunk with masked keys: their V rows (clamped copies) are left out rather than
        // weighted by 0, which an infinite V would turn into NaN; the golden never sees them.
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (kc + 4 * q + (lane >> 4) >= k_b)
#pragma unroll
                for (int e = 0; e < 8; ++e) vd[q][e] = 0.0;
    }
    __builtin_amdgcn_sched_group_barrier(0x002, 64, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 32, 1);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) st.acc[e] = mfma_f64(vd[q][e], pq[q], st.acc[e]);
}

// ---- end of a piece.

// fp64 sum of x over lanes l, l+4, l+8, l+12 of each 16-lane row (row rotations by 4 and 8).
__device__ __forceinline__ double row_quad_sum(double x) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(x));
    const int lo = static_cast<int>(u), hi = static_cast<int>(u >> 32);
    double y = x + __longlong_as_double(static_cast<long long>(
                       (static_cast<unsigned long long>(static_cast<uint32_t>(dpp_i<0x124>(hi))) << 32) |
                       static_cast<uint32_t>(dpp_i<0x124>(lo))));
    const unsigned long long v = static_cast<unsigned long long>(__double_as_longlong(y));
    const int lo2 = static_cast<int>(v), hi2 = static_cast<int>(v >> 32);
    return y + __longlong_as_double(static_cast<long long>(
                   (static_cast<unsigned long long>(static_cast<uint32_t>(dpp_i<0x128>(hi2))) << 32) |
                   static_cast<uint32_t>(dpp_i<0x128>(lo2))));
}

// Totals of a piece: the head's l summed over its 16 lanes (m_run is already common to
// them; O needs no cross-lane step, each lane owns its 8 dims over all keys).
__device__ __forceinline__ void finish_piece(PieceState& st, double& l_tot) {
    l_tot = swap_add_f64<true>(swap_add_f64<false>(row_quad_sum(st.l_run)));
}

// Element offset, within a [4][128] group of rows, of the 8 dims lane l holds.
__device__ __forceinline__ int lane_row_offset() {
    const int lane = threadIdx.x & (kWave - 1);
    return (lane & 3) * kD + out_dim_of_lane(lane);
}

// Normalise in fp64 and round double -> f32 -> BF16 (the 4 output rows of the group, in
// Q-head order, output_accumulator.v:540-686, gqa_output_collector.v:32-61).
__device__ __forceinline__ void write_rows(const DecodeArgs& a, int b, int kvh, const PieceState& st, double l_tot) {
    uint16_t o8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o8[e] = f32_to_bf16_out(static_cast<float>(st.acc[e] / l_tot));
    *reinterpret_cast<bf16x8_t*>(a.out + (static_cast<int64_t>(b) * kHq + kvh * kGroup) * kD + lane_row_offset()) =
        pack8(o8);
}

// Unnormalised partial of a piece: O (fp64) and (m, l) per head at `slot`.
__device__ __forceinline__ void write_partial(const DecodeArgs& a, int64_t slot, const PieceState& st, double l_tot) {
    const int lane = threadIdx.x & (kWave - 1);
    double2* dst = reinterpret_cast<double2*>(a.part_o + slot * kGroup * kD + lane_row_offset());
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = make_double2(st.acc[2 * j], st.acc[2 * j + 1]);
    if (lane < kGroup) a.part_ml[slot * kGroup + lane] = make_double2(st.m_run, l_tot);
}

// Agent-scope (sc1) 8-byte stores and loads: coherent across the XCDs without a cache
// write-back or invalidate (used to hand partials between workgroups inside a launch).
__device__ __forceinline__ void store_agent(unsigned long long* p, double v) {
    __hip_atomic_store(p, static_cast<unsigned long long>(__double_as_longlong(v)), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_agent(unsigned long long* p, float2 v) {
    unsigned long long u;
    __builtin_memcpy(&u, &v, 8);
    __hip_atomic_store(p, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float2 load_agent_f2(const float2* p) {
    const unsigned long long u =
        __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float2 v;
    __builtin_memcpy(&v, &u, 8);
    return v;
}

__device__ __forceinline__ double2 load_agent_d2(const double* p) {
    const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
    return make_double2(__longlong_as_double(__hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
                        __longlong_as_double(__hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
}

// Wait until every memory access this wave has issued has completed (s_waitcnt vmcnt(0)).
// A workgroup-scope release fence does not wait for global stores on gfx950, so a
// partial's stores are waited for explicitly before the counter that announces them.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// This lane's Q operands for (sequence b, KV head kvh): the group's 4 Q rows rotated at
// query_position and scaled by scale*log2(e) in double.  Two steps, so that the loads can
// be issued long before the values are needed: load_q_raw reads the 4 Q rows (lane l:
// dims l and l + 64 of each head) and the query position; build_q_operands rotates and
// scales them into LDS and reads back the lane's QOps.  sin/cos are kept while the query
// position stays the same (the 8 KV heads of a sequence).
struct QStage {
    double q[kGroup][kD];
};

struct QRaw {
    uint32_t xy[kGroup];    // head h: dim lane (low half), dim lane + 64 (high half)
    int qpos;
};

struct QRope {
    int qpos;               // position sn, cs were formed for (-1: none yet)
    double inv_freq;        // frequency of this lane's rotation pair
    double sn, cs;
};

__device__ __forceinline__ void load_q_raw(const DecodeArgs& a, int b, int kvh, QRaw& r) {
    const int lane = threadIdx.x & (kWave - 1);
    r.qpos = a.query_pos[b];
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        const uint16_t* qrow = a.q + (static_cast<int64_t>(b) * kHq + kvh * kGroup + h) * kD;
        r.xy[h] = qrow[lane] | (static_cast<uint32_t>(qrow[lane + kPairs]) << 16);
    }
}

// Rotated and scaled Q of the group into s.q (lane l: dims l and l + 64 of every head).
template <bool kRopeQ>
__device__ __forceinline__ void stage_q(const DecodeArgs& a, const QRaw& r, QRope& rope, QStage& s) {
    const int lane = threadIdx.x & (kWave - 1);
    if (kRopeQ && r.qpos != rope.qpos) {       // (uniform)
        rope_sincos(r.qpos, rope.inv_freq, rope.sn, rope.cs);
        rope.qpos = r.qpos;
    }
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        const double x = bf16_to_f32(static_cast<uint16_t>(r.xy[h] & 0xFFFFu));
        const double y = bf16_to_f32(static_cast<uint16_t>(r.xy[h] >> 16));
        double xr = x, yr = y;
        if (kRopeQ) {
            xr = x * rope.cs - y * rope.sn;
            yr = x * rope.sn + y * rope.cs;
        }
        s.q[h][lane] = xr * a.qk_scale_log2;
        s.q[h][lane + kPairs] = yr * a.qk_scale_log2;
    }
}

// QOps of lane l from a [4][128] block of rotated, scaled Q rows.
__device__ __forceinline__ void read_q_ops(const double* qs, QOps& qa) {
    const int lane = threadIdx.x & (kWave - 1);
    const double* base = qs + (lane & 3) * kD + 8 * (lane >> 4);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const double2 v = *reinterpret_cast<const double2*>(base + 32 * kb + e);
            qa.q[kb][e] = v.x;
            qa.q[kb][e + 1] = v.y;
        }
}

template <bool kRopeQ>
__device__ __forceinline__ void build_q_operands(const DecodeArgs& a, const QRaw& r, QRope& rope, QStage& s,
                                                 QOps& qa) {
    stage_q<kRopeQ>(a, r, rope, s);
    __syncthreads();
    read_q_ops(&s.q[0][0], qa);
    // (one wave: its LDS accesses run in order, so the next piece's writes need no barrier)
}

// Q operands of every (sequence, KV head), written once per call by decode_prepare_kernel
// and read by each piece: the 4 Q rows of the group rotated at query_position and scaled
// by scale*log2(e) in double, as [B][8][4][128] doubles.  One wave per (kv_head, sequence).
// It also writes the NaN rows of sequences whose lengths break the rules, and (an extra
// row of the grid) the stream-K plan.
//
// The stream-K plan (row B of the prepare grid, one wave): seq_off[b] = stream position
// of sequence b's first segment (an exclusive scan of 8 * plan_span), seq_off[B] = total
// positions, and the header {total, positions per stream workgroup, segment lead, XCD
// extra: positions moved from each odd range to its even neighbour (range_start)}.  Every
// stream workgroup finds where its range starts from these with one ballot.
__device__ __forceinline__ void build_plan(const DecodeArgs& a, int lane) {
    int64_t total, per_wg;
    int lead;
    stream_totals(a, lane, total, per_wg, lead);
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
        const int nv = b < a.batch ? plan_span(a, b, lead) : 0;
        const int64_t incl = wave_incl_scan_i64(nv, lane) + carry;
        if (b < a.batch) {
            a.seq_off[b] = (incl - nv) * kHkv;
            a.seq_nreal[b] = seq_valid_keys(a, b);
        }
        carry = __shfl(incl, kWave - 1);
    }
}

template <bool kRopeQ>
__global__ __launch_bounds__(kWave) void decode_prepare_kernel(DecodeArgs a) {
    const int kvh = blockIdx.x;
    const int b = blockIdx.y;
    const int lane = threadIdx.x;
    if (b == a.batch) {
        if (kvh == 0) build_plan(a, lane);
        return;
    }
    // The Q rows are requested together with the lengths (they exist whatever the lengths).
    QRaw raw;
    load_q_raw(a, b, kvh, raw);
    QRope rope;
    rope.qpos = -1;
    rope.inv_freq = kRopeQ ? a.rope.inv_freq[lane] : 0.0;
    rope.sn = 0.0;
    rope.cs = 1.0;
    if (seq_valid_keys(a, b) == 0) {
        if (kvh == 0) {
            uint4* out = reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(b) * kHq * kD);
            for (int i = lane; i < kHq * kD / 8; i += kWave)
                out[i] = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
        }
        return;
    }
    if (kRopeQ) rope_sincos(raw.qpos, rope.inv_freq, rope.sn, rope.cs);
    double* dst = a.q_op + (static_cast<int64_t>(b) * kHkv + kvh) * kGroup * kD;
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        const double x = bf16_to_f32(static_cast<uint16_t>(raw.xy[h] & 0xFFFFu));
        const double y = bf16_to_f32(static_cast<uint16_t>(raw.xy[h] >> 16));
        double xr = x, yr = y;
        if (kRopeQ) {
            xr = x * rope.cs - y * rope.sn;
            yr = x * rope.sn + y * rope.cs;
        }
        dst[h * kD + lane] = xr * a.qk_scale_log2;
        dst[h * kD + lane + kPairs] = yr * a.qk_scale_log2;
    }
}

// Where the rows of one piece live: segment base pointers and this lane's offsets of
// the chunk to load next (clamped to the piece's last row).
struct PieceRows {
    const char* kseg;
    const char* vseg;
    ChunkRows rows;
    uint32_t k_last;
    uint32_t v_last;
};

__device__ __forceinline__ void piece_rows(const DecodeArgs& a, int b, int kvh, int k_a, int k_b,
                                           PieceRows& r) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t head_off = static_cast<int64_t>(b) * a.kv_batch_stride +
                             static_cast<int64_t>(kvh) * a.kv_head_stride;
    r.kseg = reinterpret_cast<const char*>(a.k + head_off);
    r.vseg = reinterpret_cast<const char*>(a.v + head_off);
    const uint32_t row = static_cast<uint32_t>(a.kv_pos_stride) * 2u;   // bytes per position
    r.rows.k = static_cast<uint32_t>(k_a + (lane & 15)) * row + 16u * (lane >> 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) r.rows.v[q] = static_cast<uint32_t>(k_a + 4 * q + (lane >> 4)) * row + 16u * (lane & 15);
    r.k_last = static_cast<uint32_t>(k_b - 1) * row + 16u * (lane >> 4);
    r.v_last = static_cast<uint32_t>(k_b - 1) * row + 16u * (lane & 15);
}

__device__ __forceinline__ void load_next(PieceRows& r, uint32_t step, Chunk& c) {
    load_chunk(r.kseg, r.vseg, r.rows, r.k_last, r.v_last, c);
    advance(r.rows, step);
}

// Chunk `c` from the current piece when `in_cur`, else the first chunk of the next piece
// (the condition is wave-uniform; both addresses are formed and one is selected, so
// the load itself is unconditional).  Either way rows past the piece are clamped to its
// last row.
__device__ __forceinline__ void load_cur_or_next(bool in_cur, PieceRows& cur, const PieceRows& nxt,
                                                 uint32_t step, Chunk& c) {
    const char* kp = in_cur ? cur.kseg + min(cur.rows.k, cur.k_last) : nxt.kseg + min(nxt.rows.k, nxt.k_last);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) c.kw[kb] = load_stream16(kp + 64 * kb);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const char* vp = in_cur ? cur.vseg + min(cur.rows.v[q], cur.v_last)
                                : nxt.vseg + min(nxt.rows.v[q], nxt.v_last);
        c.vw[q] = load_stream16(vp);
    }
    advance(cur.rows, step);
}

__device__ __forceinline__ void load_q_operands(const DecodeArgs& a, int b, int kvh, QOps& qa) {
    read_q_ops(a.q_op + (static_cast<int64_t>(b) * kHkv + kvh) * kGroup * kD, qa);
}

// One piece: keys [k_a, k_b) of segment (b, kvh), whose first chunk is already in c0
// and whose Q operands are in qa.  While the piece's last chunk is computed, the first
// chunk of the next piece (rows `nxt`) is requested into c0, so the wave never waits
// at a piece boundary.  Writes the output rows itself when the piece is the whole
// segment; otherwise leaves a partial for the merge kernel.  (Requesting the next piece's
// second chunk too, before this piece's end work, measured 1 % slower on long segments.)
template <bool kRopeK>
__device__ __forceinline__ void process_piece(const DecodeArgs& a, int b, int kvh, int nv, int k_a,
                                              int k_b, int64_t wg, PieceRows& cur,
                                              const PieceRows& nxt, Chunk& c0, Chunk& c1,
                                              const QOps& qa) {
    const uint32_t step = kChunk * static_cast<uint32_t>(a.kv_pos_stride) * 2u;

    PieceState st;
    init_piece(st);

    // Two register sets: chunk j+1 is in flight while chunk j is computed.  Chunk i+1
    // of an odd-length piece does not exist; its slot re-reads the piece's last row (a
    // clamped, unconditional load) and its computation is skipped, so that the next
    // piece's first chunk always lands in c0.
    const int n_chunks = (k_b - k_a + kChunk - 1) / kChunk;
    for (int i = 0;; i += 2) {
        load_cur_or_next(true, cur, nxt, step, c1);
        compute_chunk<kRopeK>(a.rope, 0, k_a + i * kChunk, k_b, c0, qa, st);
        load_cur_or_next(i + 2 < n_chunks, cur, nxt, step, c0);
        if (i + 1 < n_chunks) compute_chunk<kRopeK>(a.rope, 0, k_a + (i + 1) * kChunk, k_b, c1, qa, st);
        if (i + 2 >= n_chunks) break;
    }

    double l_tot;
    finish_piece(st, l_tot);
    if (k_a == 0 && k_b == nv) {
        write_rows(a, b, kvh, st, l_tot);      // the whole segment
        return;
    }
    write_partial(a, wg + static_cast<int64_t>(b) * kHkv + kvh, st, l_tot);
}
// Per-sequence key offsets for 64 sequences at a time, one per lane: o = seq_off[base +
// lane], o1 = seq_off[base + lane + 1] (the segments of sequence b hold keys [o, o1)).
struct SeqWindow {
    int base;
    int64_t o;
    int64_t o1;
    int nreal;        // planned windows: keys that count (less than o1 - o for a paged cache)
    int lead;         // stream positions before each segment's first key (uniform)
};

__device__ __forceinline__ void load_seq_window(const DecodeArgs& a, int base, SeqWindow& sw) {
    const int bb = base + static_cast<int>(threadIdx.x & (kWave - 1));
    sw.base = base;
    sw.o = bb < a.batch ? a.seq_off[bb] : INT64_MAX;
    sw.o1 = bb < a.batch ? a.seq_off[bb + 1] : INT64_MAX;
    sw.nreal = bb < a.batch ? a.seq_nreal[bb] : 0;
}

// The segment after (b, kvh) that has keys: the next KV head of b, or KV head 0 of the
// next sequence with keys.  Returns false when there is none (possible only if the
// lengths changed while the kernel ran).
__device__ __forceinline__ bool next_segment(const DecodeArgs& a, SeqWindow& sw, int& b, int& kvh,
                                             int& nv) {
    if (kvh + 1 < kHkv) {
        ++kvh;
        return true;
    }
    kvh = 0;
    while (true) {
        const int bb = sw.base + static_cast<int>(threadIdx.x & (kWave - 1));
        const uint64_t m = __ballot(bb < a.batch && bb > b && sw.o1 > sw.o);
        if (m) {
            const int j = __ffsll(static_cast<unsigned long long>(m)) - 1;
            b = sw.base + j;
            nv = static_cast<int>((__shfl(sw.o1, j) - __shfl(sw.o, j)) / kHkv) - sw.lead;
            return true;
        }
        if (sw.base + kWave >= a.batch) return false;
        load_seq_window(a, sw.base + kWave, sw);
    }
}

template <bool kRopeK>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(1))) void decode_stream_kernel(DecodeArgs a) {
    // The first window of sequence offsets does not depend on the plan header: both are
    // requested at once.
    SeqWindow w0;
    load_seq_window(a, 0, w0);
    const int64_t w = blockIdx.x;
    const int64_t total = a.plan_hdr[0];
    const int64_t per_wg = a.plan_hdr[1];
    const int lead = static_cast<int>(a.plan_hdr[2]);
    const int64_t extra = a.plan_hdr[3];
    int64_t x = range_start(per_wg, extra, w);
    if (x >= total) return;
    const int64_t x_end = min(range_start(per_wg, extra, w + 1), total);

    // Start sequence b = the last b with seq_off[b] <= x (it has keys, since x < total).
    SeqWindow sw;
    int b = 0;
    int64_t off = 0, next = 0;
    for (int base = 0; base < a.batch; base += kWave) {
        SeqWindow t = w0;
        if (base > 0) load_seq_window(a, base, t);
        const uint64_t le = __ballot(t.o <= x);
        if (le) {
            const int j = 63 - __clzll(static_cast<long long>(le));
            b = base + j;
            off = __shfl(t.o, j);
            next = __shfl(t.o1, j);
            sw = t;
        }
    }
    sw.lead = lead;
    int kvh, key, nvb;
    locate_first_piece(off, next, lead, x, kvh, key, nvb);
    x = uniform_i64(x);
    b = __builtin_amdgcn_readfirstlane(b);
    kvh = __builtin_amdgcn_readfirstlane(kvh);
    key = __builtin_amdgcn_readfirstlane(key);
    nvb = __builtin_amdgcn_readfirstlane(nvb);
    int k_b = __builtin_amdgcn_readfirstlane(
        static_cast<int>(min(static_cast<int64_t>(nvb), key + (x_end - x))));

    const uint32_t step = kChunk * static_cast<uint32_t>(a.kv_pos_stride) * 2u;
    PieceRows cur;
    piece_rows(a, b, kvh, key, k_b, cur);
    Chunk c0, c1;
    load_next(cur, step, c0);
    QOps qa;
    load_q_operands(a, b, kvh, qa);

    while (true) {
        // The next piece of this range (or, after the last one, a re-read of this piece's
        // last row), whose first chunk and Q operands are requested during this piece.
        // x_next is the end of this segment's span when the piece reaches it; the range has
        // a piece of the next segment if it reaches that segment's first key.
        const int64_t x_next = x + (k_b - key);
        int b2 = b, kvh2 = kvh, nv2 = nvb, key2 = k_b - 1, k_b2 = k_b;
        bool more = x_next + lead < x_end;
        if (more) {
            more = next_segment(a, sw, b2, kvh2, nv2);
            b2 = __builtin_amdgcn_readfirstlane(b2);
            kvh2 = __builtin_amdgcn_readfirstlane(kvh2);
            nv2 = __builtin_amdgcn_readfirstlane(nv2);
            key2 = 0;
            k_b2 = __builtin_amdgcn_readfirstlane(
                static_cast<int>(min(static_cast<int64_t>(nv2), x_end - x_next - lead)));
        }
        if (!more) {
            b2 = b;
            kvh2 = kvh;
            nv2 = nvb;
            key2 = k_b - 1;
            k_b2 = k_b;
        }
        PieceRows nxt;
        piece_rows(a, b2, kvh2, key2, k_b2, nxt);
        QOps qa2;
        load_q_operands(a, b2, kvh2, qa2);

        process_piece<kRopeK>(a, b, kvh, nvb, key, k_b, w, cur, nxt, c0, c1, qa);
        if (!more) break;

        x = x_next + lead;
        b = b2;
        kvh = kvh2;
        nvb = nv2;
        key = key2;
        k_b = k_b2;
        cur = nxt;
        advance(cur.rows, step);     // its first chunk is in c0 already
        qa = qa2;
    }
}


// ---------------------------------------------------------------------------------
// Paged cache (block tables).  The pool holds blocks of 16 positions -- the reference
// core's KV_BLOCK_LEN (gqa_controller.v:20) -- and block j of sequence b is pool block
// block_table[b][j]; block id, KV head and position address a row as
// id*block_stride + h*head_stride + p*pos_stride.  The stream-K key space pads every
// segment to whole blocks, so each piece starts on a block and each 16-key chunk is one
// (block, KV head): 4 KB of K and 4 KB of V at one place.  Block ids are requested two
// chunks ahead of the chunk that needs them.  An id outside [0, n_blocks) reads block 0
// instead and turns that sequence's rows into NaN (never an out-of-range read).

// Block id of block j of sequence b, as a (lane-uniform) vector load: its value is made
// scalar only where it is used, so that waiting for it never waits for loads issued
// after it.
__device__ __forceinline__ int load_block_id(const DecodeArgs& a, int b, int j) {
    return a.block_table[static_cast<int64_t>(b) * a.max_blocks + j];
}

// Pool element offset of (block id, KV head kvh); ids outside the pool read block 0 and
// clear `ok`.
__device__ __forceinline__ int64_t page_elem(const DecodeArgs& a, int id_vgpr, int kvh, bool& ok) {
    const int pid = __builtin_amdgcn_readfirstlane(id_vgpr);
    ok = pid >= 0 && pid < a.n_blocks;
    return static_cast<int64_t>(ok ? pid : 0) * a.kv_batch_stride + static_cast<int64_t>(kvh) * a.kv_head_stride;
}

// K and V rows of one block-chunk (the Chunk lane layout): lane rows clamped to the chunk's
// last valid row.
__device__ __forceinline__ void load_page_chunk(const DecodeArgs& a, int64_t elem, int rows_valid, Chunk& c) {
    const int lane = threadIdx.x & (kWave - 1);
    const char* kp = reinterpret_cast<const char*>(a.k + elem);
    const char* vp = reinterpret_cast<const char*>(a.v + elem);
    const uint32_t row = static_cast<uint32_t>(a.kv_pos_stride) * 2u;
    const int r_last = rows_valid - 1;
    const char* krow = kp + static_cast<uint32_t>(min(lane & 15, r_last)) * row + 16u * (lane >> 4);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) c.kw[kb] = load_stream16(krow + 64 * kb);
#pragma unroll
    for (int q = 0; q < 4; ++q)
        c.vw[q] = load_stream16(vp + static_cast<uint32_t>(min(4 * q + (lane >> 4), r_last)) * row + 16u * (lane & 15));
}

// A piece of the paged stream: segment (b, kvh), keys [k_a, k_b) of nvp block-padded keys
// (kend = the piece's last real key + 1).  Its first chunk is loaded before it starts (by
// the previous piece, or the kernel's prologue), with the id of its second block.
struct PagePiece {
    int b, kvh, nvp, k_a, k_b, kend;
    int id1;          // block id (vector register) of the piece's second block (clamped)
    bool ok;          // the first chunk's block id was valid
};

// The first chunk of piece `p` (block k_a/16 of sequence p.b, id `id0`) into c; returns
// whether the id was valid.
__device__ __forceinline__ bool load_first_page_chunk(const DecodeArgs& a, const PagePiece& p, int id0, Chunk& c) {
    bool ok;
    const int j0 = p.k_a / kChunk;
    load_page_chunk(a, page_elem(a, id0, p.kvh, ok), max(1, min(kChunk, p.kend - j0 * kChunk)), c);
    return ok;
}

// One piece whose first chunk is in c0.  The last iteration's second load fetches the first
// chunk of `nx` (when has_next; its first block id nx_id0) into c0 -- so that the next
// piece never waits for its first data -- and sets nx.ok.
template <bool kRopeK>
__device__ __forceinline__ void process_page_piece(const DecodeArgs& a, const PagePiece& p, int64_t wg, Chunk& c0,
                                                   Chunk& c1, const QOps& qa, bool has_next, PagePiece& nx,
                                                   int nx_id0) {
    const int b = p.b, kvh = p.kvh, k_a = p.k_a, kend = p.kend;
    PieceState st;
    init_piece(st);
    bool all_ok = p.ok;
    if (k_a < kend) {
        const int j0 = k_a / kChunk;
        const int jn = (kend - 1) / kChunk;    // last block holding a key of this piece
        const int n_chunks = jn - j0 + 1;
        bool ok;
        // Block ids are requested two chunks ahead of the chunk whose loads need them, each
        // before that iteration's data loads: waiting for one never waits for data that
        // is still meant to be in flight.
        int id_next = p.id1;
        // One exit, at the end: chunks past the piece's last re-read its last block (or,
        // for the last one, fetch the next piece's first chunk) and are not computed, so
        // that every path into the loop head has the same loads in flight.
        for (int i = 0;; i += 2) {
            {
                const int j = min(j0 + i + 1, jn);
                const int id_after = load_block_id(a, b, min(j + 1, jn));
                load_page_chunk(a, page_elem(a, id_next, kvh, ok), min(kChunk, kend - j * kChunk), c1);
                all_ok = all_ok && ok;
                id_next = id_after;
            }
            compute_chunk<kRopeK>(a.rope, 0, k_a + i * kChunk, kend, c0, qa, st);
            {
                const bool last = i + 2 >= n_chunks;
                const bool to_next = last && has_next;
                const int j = min(j0 + i + 2, jn);
                const int id_after = load_block_id(a, b, min(j + 1, jn));
                const int nj0 = nx.k_a / kChunk;
                load_page_chunk(a, page_elem(a, to_next ? nx_id0 : id_next, to_next ? nx.kvh : kvh, ok),
                                to_next ? max(1, min(kChunk, nx.kend - nj0 * kChunk)) : min(kChunk, kend - j * kChunk),
                                c0);
                if (to_next)
                    nx.ok = ok;
                else
                    all_ok = all_ok && ok;
                id_next = id_after;
            }
            if (i + 1 < n_chunks) compute_chunk<kRopeK>(a.rope, 0, k_a + (i + 1) * kChunk, kend, c1, qa, st);
            if (i + 2 >= n_chunks) break;
        }
    } else if (has_next) {
        nx.ok = load_first_page_chunk(a, nx, nx_id0, c0);   // a piece of padding only
    }
    double l_tot;
    finish_piece(st, l_tot);
    if (!all_ok) {
        // an invalid block id: poison the sequence's rows of this segment
        st.m_run = 0.0;
        l_tot = __longlong_as_double(0x7ff8000000000000ll);
    }
    if (k_a == 0 && p.k_b == p.nvp) {
        write_rows(a, b, kvh, st, l_tot);      // the whole segment
        return;
    }
    write_partial(a, wg + static_cast<int64_t>(b) * kHkv + kvh, st, l_tot);
}

template <bool kRopeK>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(1))) void decode_paged_stream_kernel(DecodeArgs a) {
    const int64_t w = blockIdx.x;
    const int64_t total = a.plan_hdr[0];
    const int64_t per_wg = a.plan_hdr[1];
    const int lead = static_cast<int>(a.plan_hdr[2]);
    const int64_t extra = a.plan_hdr[3];
    int64_t x = range_start(per_wg, extra, w);
    if (x >= total) return;
    const int64_t x_end = min(range_start(per_wg, extra, w + 1), total);

    // Start sequence: the last b with seq_off[b] <= x (it has keys, since x < total).
    SeqWindow sw;
    int b = 0;
    int64_t off = 0, next = 0;
    for (int base = 0; base < a.batch; base += kWave) {
        SeqWindow t;
        load_seq_window(a, base, t);
        const uint64_t le = __ballot(t.o <= x);
        if (le) {
            const int j = 63 - __clzll(static_cast<long long>(le));
            b = base + j;
            off = __shfl(t.o, j);
            next = __shfl(t.o1, j);
            sw = t;
        }
    }
    PagePiece cur;
    {
        sw.lead = lead;
        int kvh, key, nvp;
        locate_first_piece(off, next, lead, x, kvh, key, nvp);
        x = uniform_i64(x);
        cur.b = __builtin_amdgcn_readfirstlane(b);
        cur.nvp = __builtin_amdgcn_readfirstlane(nvp);
        cur.kvh = __builtin_amdgcn_readfirstlane(kvh);
        cur.k_a = __builtin_amdgcn_readfirstlane(key);
    }
    cur.k_b = __builtin_amdgcn_readfirstlane(
        static_cast<int>(min(static_cast<int64_t>(cur.nvp), cur.k_a + (x_end - x))));
    cur.kend = min(cur.k_b, __builtin_amdgcn_readfirstlane(__shfl(sw.nreal, cur.b - sw.base)));
    {
        const int j0 = cur.k_a / kChunk;
        const int jn = max(j0, (cur.kend - 1) / kChunk);
        cur.id1 = load_block_id(a, cur.b, min(j0 + 1, jn));
        cur.ok = true;
    }
    Chunk c0, c1;
    if (cur.k_a < cur.kend) cur.ok = load_first_page_chunk(a, cur, load_block_id(a, cur.b, cur.k_a / kChunk), c0);
    QOps qa;
    load_q_operands(a, cur.b, cur.kvh, qa);

    while (true) {
        // The next piece of this range, and everything it needs before its first chunk
        // (its length, first two block ids, Q operands), requested during this piece.
        const int64_t x_next = x + (cur.k_b - cur.k_a);   // as in decode_stream_kernel
        PagePiece nx = cur;
        int b2 = cur.b, kvh2 = cur.kvh, nv2 = cur.nvp;
        bool more = x_next + lead < x_end;
        if (more) more = next_segment(a, sw, b2, kvh2, nv2);
        int nx_id0 = cur.id1;
        QOps qa2;
        if (more) {
            nx.b = __builtin_amdgcn_readfirstlane(b2);
            nx.kvh = __builtin_amdgcn_readfirstlane(kvh2);
            nx.nvp = __builtin_amdgcn_readfirstlane(nv2);
            nx.k_a = 0;
            nx.k_b = __builtin_amdgcn_readfirstlane(
                static_cast<int>(min(static_cast<int64_t>(nx.nvp), x_end - x_next - lead)));
            nx.kend = min(nx.k_b, __builtin_amdgcn_readfirstlane(__shfl(sw.nreal, nx.b - sw.base)));
            const int jn2 = max(0, (nx.kend - 1) / kChunk);
            nx_id0 = load_block_id(a, nx.b, 0);
            nx.id1 = load_block_id(a, nx.b, min(1, jn2));
            nx.ok = true;
            load_q_operands(a, nx.b, nx.kvh, qa2);
        }
        process_page_piece<kRopeK>(a, cur, w, c0, c1, qa, more, nx, nx_id0);
        if (!more) break;
        x = x_next + lead;
        cur = nx;
        qa = qa2;
    }
}

// Merge the pieces of multi-piece segments: one 4-wave workgroup per (KV head,
// sequence), wave h for Q head 4*kvh + h.  Slots w + seg for w in [w_first, w_last]
// hold the pieces of segment seg; their (m, l) are read one per lane, the weights
// 2^(m - max) are exact, O is summed in fp64 two dims per lane, and the row is
// rounded double -> f32 -> BF16.  Segments held by one workgroup were written by the
// stream kernel and are skipped.
__global__ __launch_bounds__(kGroup * kWave) void decode_merge_kernel(DecodeArgs a) {
    const int kvh = blockIdx.x;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1);
    const int h = threadIdx.x / kWave;
    const int64_t per_wg = a.plan_hdr[1];
    const int64_t off = a.seq_off[b];
    const int span = static_cast<int>((a.seq_off[b + 1] - off) / kHkv);
    if (span == 0) return;
    const int lead = static_cast<int>(a.plan_hdr[2]);
    const int nv = span - lead;
    const int64_t seg_off = off + static_cast<int64_t>(kvh) * span + lead;   // stream position of key 0
    const int64_t extra = a.plan_hdr[3];
    const int64_t w_first = range_of(per_wg, extra, seg_off);
    const int n_pieces = static_cast<int>(range_of(per_wg, extra, seg_off + nv - 1) - w_first) + 1;
    if (n_pieces == 1) return;
    const int64_t slot0 = w_first + static_cast<int64_t>(b) * kHkv + kvh;

    // Pieces in passes of 64, one (m, l) per lane; the O rows of a pass are requested
    // together with its (m, l) (indices clamped to the last piece, whose extra copies get
    // weight 0) and weighted by 2^(m - running max) once the pass's max is known.
    double mx = -INFINITY;
    double l = 0.0, o0 = 0.0, o1 = 0.0;
    for (int p0 = 0; p0 < n_pieces; p0 += kWave) {
        const int cnt = min(kWave, n_pieces - p0);
        const int p = p0 + min(lane, cnt - 1);
        const double2 ml = a.part_ml[(slot0 + p) * kGroup + h];
        for (int q = 0; q < cnt; q += 8) {
            double2 o[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int qq = min(q + u, cnt - 1);
                o[u] = reinterpret_cast<const double2*>(
                    a.part_o + ((slot0 + p0 + qq) * kGroup + h) * kD)[lane];
            }
            if (q == 0) {
                // New running max over this pass; rescale what earlier passes summed.
                const double m_pass = wave_max_f64(lane < cnt ? ml.x : -INFINITY);
                const double m_new = fmax(mx, m_pass);
                if (mx != -INFINITY && m_new != mx) {
                    const int e = max_shift_f64(mx, m_new);
                    l = ldexp(l, e);
                    o0 = ldexp(o0, e);
                    o1 = ldexp(o1, e);
                }
                mx = m_new;
                if (lane < cnt && ml.x != -INFINITY) l += ldexp(ml.y, max_shift_f64(ml.x, mx));
            }
            // a piece holding no key (padding of a paged segment) has m = -inf: weight 0
            const int e_lane = lane < cnt && ml.x != -INFINITY ? max_shift_f64(ml.x, mx) : -1100;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int ee = __shfl(e_lane, min(q + u, kWave - 1));
                if (q + u < cnt) {
                    o0 += ldexp(o[u].x, ee);
                    o1 += ldexp(o[u].y, ee);
                }
            }
        }
    }
    l += __shfl_xor(l, 1);
    l += __shfl_xor(l, 2);
    l += __shfl_xor(l, 4);
    l += __shfl_xor(l, 8);
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    uint32_t* out = reinterpret_cast<uint32_t*>(
        a.out + (static_cast<int64_t>(b) * kHq + kvh * kGroup + h) * kD);
    const uint32_t lo = f32_to_bf16_out(static_cast<float>(o0 / l));
    const uint32_t hi = f32_to_bf16_out(static_cast<float>(o1 / l));
    out[lane] = lo | (hi << 16);
}


// ---------------------------------------------------------------------------------
// Single-launch decode for small batches (few keys in all, where three dependent launches
// would cost more than the HBM traffic).  One 4-wave workgroup per (piece, segment);
// a piece is a.piece_keys keys, a quarter per wave.  The workgroup prepares the group's
// Q operands once (wave h rotates head h), each wave streams its quarter like a
// stream-kernel piece, the four wave states are combined in LDS, and the piece either
// writes the output rows (a one-piece segment) or leaves its partial; the last piece of
// a segment to finish merges them, one wave per head.  Partials are written and read
// with agent-scope (sc1) accesses, which go through to memory past the XCD-local L2s,
// and the per-segment counter is a device-scope atomic incremented only after the
// partial's stores have completed.  The merging piece resets the counter, so a
// workspace needs zeroing (gqa_decode_workspace_init) before its first use only.

constexpr int kSingleWaves = 4;

template <bool kRopeQ, bool kRopeK>
__global__ __launch_bounds__(kSingleWaves * kWave) void decode_single_kernel(DecodeArgs a) {
    __shared__ double q_s[kGroup][kD];
    __shared__ double o_s[kSingleWaves][kGroup][kD];     // each wave's O (blocks summed)
    __shared__ double m_s[kSingleWaves][kGroup];
    __shared__ double l_s[kSingleWaves][kGroup];
    __shared__ int last_s;
    const int piece = blockIdx.x;
    const int seg = blockIdx.y;
    const int b = seg / kHkv;
    const int kvh = seg % kHkv;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int nv = seq_valid_keys(a, b);
    if (nv == 0) {
        if (kvh == 0 && piece == 0) {
            uint4* out = reinterpret_cast<uint4*>(a.out + static_cast<int64_t>(b) * kHq * kD);
            for (int i = threadIdx.x; i < kHq * kD / 8; i += kSingleWaves * kWave)
                out[i] = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
        }
        return;
    }
    const int n_pieces = (nv + a.piece_keys - 1) / a.piece_keys;
    if (piece >= n_pieces) return;                       // uniform over the workgroup
    const int quarter = a.piece_keys / kSingleWaves;
    const int k_a = min(nv, piece * a.piece_keys + wave * quarter);
    const int k_b = min(nv, k_a + quarter);
    const bool busy = k_a < k_b;                         // uniform over the wave

    // First chunk of this wave's quarter, requested before the Q operands are formed.
    PieceRows cur;
    piece_rows(a, b, kvh, busy ? k_a : nv - 1, busy ? k_b : nv, cur);
    const uint32_t step = kChunk * static_cast<uint32_t>(a.kv_pos_stride) * 2u;
    Chunk c0, c1;
    load_next(cur, step, c0);

    // Q operands: wave h rotates and scales Q head 4*kvh + h into q_s; every wave then
    // reads its QOps back.
    {
        const int qpos = a.query_pos[b];
        double sn = 0.0, cs = 1.0;
        if (kRopeQ) rope_sincos(qpos, a.rope.inv_freq[lane], sn, cs);
        const uint16_t* qrow = a.q + (static_cast<int64_t>(b) * kHq + kvh * kGroup + wave) * kD;
        const double x = bf16_to_f32(qrow[lane]);
        const double y = bf16_to_f32(qrow[lane + kPairs]);
        double xr = x, yr = y;
        if (kRopeQ) {
            xr = x * cs - y * sn;
            yr = x * sn + y * cs;
        }
        q_s[wave][lane] = xr * a.qk_scale_log2;
        q_s[wave][lane + kPairs] = yr * a.qk_scale_log2;
    }
    __syncthreads();
    QOps qa;
    read_q_ops(&q_s[0][0], qa);

    PieceState st;
    init_piece(st);
    if (busy) {
        const int n_chunks = (k_b - k_a + kChunk - 1) / kChunk;
        for (int i = 0;; i += 2) {
            load_next(cur, step, c1);
            compute_chunk<kRopeK>(a.rope, 0, k_a + i * kChunk, k_b, c0, qa, st);
            if (i + 1 >= n_chunks) break;
            load_next(cur, step, c0);
            compute_chunk<kRopeK>(a.rope, 0, k_a + (i + 1) * kChunk, k_b, c1, qa, st);
            if (i + 2 >= n_chunks) break;
        }
    }
    double l_tot;
    finish_piece(st, l_tot);
#pragma unroll
    for (int e = 0; e < 8; ++e) (&o_s[wave][0][0])[lane_row_offset() + e] = st.acc[e];
    if (lane < kGroup) {
        m_s[wave][lane] = st.m_run;
        l_s[wave][lane] = l_tot;
    }
    __syncthreads();

    // Wave h combines head h over the four quarters: lane owns dims 2*lane, 2*lane + 1.
    const int h = wave;
    double mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSingleWaves; ++w) mx = fmax(mx, m_s[w][h]);
    double l = 0.0, o0 = 0.0, o1 = 0.0;
#pragma unroll
    for (int w = 0; w < kSingleWaves; ++w) {
        const double m = m_s[w][h];
        if (m == -INFINITY) continue;                    // an idle quarter
        const int e = max_shift_f64(m, mx);
        l += ldexp(l_s[w][h], e);
        o0 += ldexp(o_s[w][h][2 * lane], e);
        o1 += ldexp(o_s[w][h][2 * lane + 1], e);
    }
    uint32_t* orow = reinterpret_cast<uint32_t*>(a.out + (static_cast<int64_t>(b) * kHq + kvh * kGroup + h) * kD);
    if (n_pieces == 1) {
        orow[lane] = f32_to_bf16_out(static_cast<float>(o0 / l)) |
                     (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(o1 / l))) << 16);
        return;
    }
    const int64_t slot0 = static_cast<int64_t>(seg) * a.pieces_cap;
    // Publish the partial with agent-scope stores (written through the XCD's L2, which is
    // not coherent with the other XCDs'), and wait until they have completed before the
    // counter is touched: a __threadfence here would write back the whole L2 instead.
    // The counter's atomic returns only after it is performed, and the merge's agent-scope
    // loads are issued after that.  The hardware order comes from the waits (vmcnt(0)
    // before the count, the atomic's return value before any merge load); the signal
    // fences and the barriers keep the compiler from moving a store below the count or a
    // load above it.
    {
        unsigned long long* po =
            reinterpret_cast<unsigned long long*>(a.part_o + ((slot0 + piece) * kGroup + h) * kD) + 2 * lane;
        store_agent(po, o0);
        store_agent(po + 1, o1);
        if (lane == 0) {
            unsigned long long* pml = reinterpret_cast<unsigned long long*>(a.part_ml + (slot0 + piece) * kGroup + h);
            store_agent(pml, mx);
            store_agent(pml + 1, l);
        }
        wait_vmem();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    __syncthreads();
    // Count finished pieces (device-scope atomic); the last piece merges and resets the
    // counter for the next call on this workspace.
    if (threadIdx.x == 0) last_s = atomicAdd(&a.seg_count[seg], 1ull) == static_cast<unsigned long long>(n_pieces - 1);
    __syncthreads();
    if (!last_s) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (threadIdx.x == 0) __hip_atomic_store(&a.seg_count[seg], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // Merge the segment's pieces, wave h for head h (lane owns dims 2*lane, 2*lane + 1), in
    // piece order.  Up to 16 pieces: every (m, l) and O row requested at once.  More: the
    // (m, l) of 64 pieces per pass, one per lane, first, then the O rows 16 at a time.
    l = 0.0;
    o0 = 0.0;
    o1 = 0.0;
    if (n_pieces <= 16) {
        // lane u < 16 holds piece u's (m, l) (copies of the last piece past n_pieces)
        double2 ov[16];
        const double2 mlu = load_agent_d2(reinterpret_cast<const double*>(
            a.part_ml + (slot0 + min(lane & 15, n_pieces - 1)) * kGroup + h));
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int p = min(u, n_pieces - 1);
            ov[u] = load_agent_d2(a.part_o + ((slot0 + p) * kGroup + h) * kD + 2 * lane);
        }
        const double m_all = wave_max_f64(mlu.x);     // copies of the last piece add nothing
        const int e_l = (lane & 15) < n_pieces ? max_shift_f64(mlu.x, m_all) : -1100;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int e = __shfl(e_l, u);
            l += ldexp(__shfl(mlu.y, u), e);
            o0 += ldexp(ov[u].x, e);
            o1 += ldexp(ov[u].y, e);
        }
    } else {
        double m_all = -INFINITY;
        for (int p0 = 0; p0 < n_pieces; p0 += kWave) {
            const int p = p0 + lane;
            m_all = fmax(m_all, p < n_pieces ? load_agent_d2(reinterpret_cast<const double*>(
                                                   a.part_ml + (slot0 + p) * kGroup + h)).x
                                             : -INFINITY);
        }
        m_all = wave_max_f64(m_all);
        for (int p0 = 0; p0 < n_pieces; p0 += 16) {
            double2 ov[16];
            double2 ml[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int p = min(p0 + u, n_pieces - 1);
                ov[u] = load_agent_d2(a.part_o + ((slot0 + p) * kGroup + h) * kD + 2 * lane);
                ml[u] = load_agent_d2(reinterpret_cast<const double*>(a.part_ml + (slot0 + p) * kGroup + h));
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                // copies of the last piece (indices clamped above) get weight 0
                const int e = p0 + u < n_pieces ? max_shift_f64(ml[u].x, m_all) : -1100;
                l += ldexp(ml[u].y, e);
                o0 += ldexp(ov[u].x, e);
                o1 += ldexp(ov[u].y, e);
            }
        }
    }
    orow[lane] = f32_to_bf16_out(static_cast<float>(o0 / l)) |
                 (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(o1 / l))) << 16);
}

// ---------------------------------------------------------------------------------
// fp64 rescore of the output rows a prefill or multi-token call flags.  Their MFMA kernels
// carry scores in fp32 (Q in split parts against BF16 or staged fp16 K); an output element
// that cancels to near zero can then miss 64 BF16 ULP of the golden's double value, so the
// flag (rs_flag_decide, in the prefill attention epilogue or the multi-token merge) marks every row
// holding an element that may lie within the kernels' error of zero, and rescore_kernel
// recomputes the flagged rows in fp64 throughout (scores, exp2 and weighted V): the
// one-token golden step at position start + t over keys 0 .. start + t, the chunk's own keys
// rotated in double from the new K rows and not re-rounded, as the golden rotates K
// (pyfiles/gen_gqa_wrapper_vectors.py:121-139).
//
// The flagged rows of one (sequence, KV head) read the same K/V rows, so they are taken four
// at a time ("tiles", in flagging order) as the four columns of the decode kernels' fp64 MFMA
// chunk (v_mfma_f64_4x4x4_4b: 16 keys x 4 columns per chunk, each K/V row read once for the
// four): column c is row c of the tile, with its own Q (rotated at its own position) and its
// own last key start + t (later keys score -inf, p = 0 exactly).  The columns do not mix: a
// row's arithmetic is the same whichever rows share its tile.
//
// A persistent grid of one-wave workgroups takes (tile, piece) pairs; piece p of a tile's
// np pieces takes its 16-key chunks p, p + np, p + 2 np, ... (so every piece of a tile has
// about the same work whatever its rows' lengths), two chunks ahead in flight.  np follows
// from the tile count, the partial slots and the capacity only -- the flagged rows' count
// per (sequence, KV head) and the call's sizes, never the order rows were flagged in -- so
// the results are bit-for-bit repeatable.  A piece's partial (fp64 O, running max and sum
// per column) is published with agent-scope stores and the tile's last piece merges them
// (the pieces' (m, l) one piece per lane, their O eight pieces at a time), as in
// decode_single_kernel.

// Rows path (the flagged rows spread thin over their (sequence, KV head) pairs): one row per
// wave, fp64 VALU (an fp64 MFMA would compute four columns for one and costs more than the
// VALU chain for a single row) -- lane l holds key slot l/8 of an 8-key chunk and the 16
// dims {8c + i, 64 + 8c + i : i < 8}, c = l % 8 -- 8 rotate_half pairs, so a chunk key's
// rotation is lane-local.  A key's score is the sum over its eight lanes; each lane
// accumulates p * V over its own keys for its 16 dims, and the 8 key slots are summed once
// per piece.  A persistent grid of one-wave workgroups takes (row, piece) pairs, piece p of
// a row taking its chunks p, p + n_pieces, ..., so that the pieces share the costlier chunk
// keys evenly.  With at most 64 flagged rows (one per lane) every workgroup reads all of them
// and gives each row pieces in proportion to its chunks (at least kRsMinChunks per piece, at
// most kRsMaxPieces pieces): the longest row, which sets the kernel's time, gets the most.
// With more rows each gets gridDim / rows pieces.  A row's result depends on its keys and
// its piece count only, which follow from the flagged rows' key counts and the grid, never
// from the order they were flagged in.

constexpr int kRsKeys = 8;              // keys per rescore chunk (one per 8 lanes)
constexpr int kRsMinChunks = 4;         // chunks per piece at least (proportional split)
constexpr int kRsMergeBatch = 32;       // partials loaded at once by a row's merge

// This lane's 16 dims of one K row and one V row (BF16): x dims 8c .. 8c+7, y dims 64 + 8c ..
struct RsRows {
    uint4 kx, ky, vx, vy;
};

// Plain (cached) loads, unlike the stream kernels' nontemporal ones: the flagged rows of one
// (sequence, KV head) run at the same time and read the same K/V rows, so the second row's
// reads hit the caches (config 5: 59 -> 54 us).
__device__ __forceinline__ void rs_load(const char* krow, const char* vrow, RsRows& r) {
    const int c = threadIdx.x & 7;
    r.kx = *reinterpret_cast<const uint4*>(krow + 16 * c);
    r.ky = *reinterpret_cast<const uint4*>(krow + 2 * kPairs + 16 * c);
    r.vx = *reinterpret_cast<const uint4*>(vrow + 16 * c);
    r.vy = *reinterpret_cast<const uint4*>(vrow + 2 * kPairs + 16 * c);
}

// (cos, sin) of this lane's 8 frequencies 8c + i from a cos/sin row (64 pairs).
__device__ __forceinline__ void rs_load_cs(const double2* cs_row, double2 (&cs)[8]) {
    const double2* p = cs_row + 8 * (threadIdx.x & 7);
#pragma unroll
    for (int i = 0; i < 8; ++i) cs[i] = p[i];
}

// 8 BF16 values -> double (exact).
__device__ __forceinline__ void rs_widen(const uint4& w, double* d) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        d[2 * j] = static_cast<double>(__uint_as_float(u[j] << 16));
        d[2 * j + 1] = static_cast<double>(__uint_as_float(u[j] & 0xffff0000u));
    }
}

// Sum over the eight lanes of a key slot (lanes 8j .. 8j+7), the same bits in all eight:
// within quads by DPP lane swaps, then across the two quads.
__device__ __forceinline__ double rs_slot_sum(double x) {
    int lo = __double2loint(x), hi = __double2hiint(x);
    x += __hiloint2double(__builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, false),
                          __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, false));     // quad_perm 1,0,3,2
    lo = __double2loint(x);
    hi = __double2hiint(x);
    x += __hiloint2double(__builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, false),
                          __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, false));     // quad_perm 2,3,0,1
    return x + __shfl_xor(x, 4);
}

// Running state of a piece: this lane's O over its keys (its 16 dims), the sum of p over
// its keys (each key counted in all eight of its lanes) and the wave's running max, in
// double: the rows sent here include rows whose scores are far beyond 2^24, where an fp32
// max could not sit within a few units of the largest score (and p of that key would
// underflow).
struct RsState {
    double o[16];
    double l;
    double m;
};

// Lazy running max (integer-valued, wave-uniform): raised to the ceiling of the largest
// score when one exceeds it by more than kMaxHeadroom; O and l move by an exact power of 2.
template <int G>
__device__ __forceinline__ void rs_raise_max(const double (&s)[G], RsState& st) {
    bool grow = false;
#pragma unroll
    for (int g = 0; g < G; ++g) grow |= s[g] > st.m + kMaxHeadroom;
    if (__ballot(grow)) {
        double cm = s[0];
#pragma unroll
        for (int g = 1; g < G; ++g) cm = fmax(cm, s[g]);
        cm = fmax(cm, dpp_d<0x128>(cm));                      // key slots 8 lanes apart
        cm = swap_max_f64<true>(swap_max_f64<false>(cm));
        const double m_new = ceil(cm);
        const int shift = (st.m == -INFINITY) ? 0 : max_shift_f64(st.m, m_new);
#pragma unroll
        for (int i = 0; i < 16; ++i) st.o[i] = ldexp(st.o[i], shift);
        st.l = ldexp(st.l, shift);
        st.m = m_new;
    }
}

// G chunks at once (their score, exp2 and weighted-V chains interleave): one key per 8
// lanes in each (valid[g]: inside the row's keys); kRot: K rotated with cs first.  The
// chunks are accumulated in order g = 0, 1, ...
template <int G, bool kRot>
__device__ __forceinline__ void rs_chunks(const RsRows* r, const double (&q)[16], const bool (&valid)[G],
                                          const double2 (*cs)[8], RsState& st) {
    double sa[G], sb[G];
#pragma unroll
    for (int g = 0; g < G; ++g) sa[g] = sb[g] = 0.0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        double k[16];
        rs_widen(r[g].kx, k);
        rs_widen(r[g].ky, k + 8);
        if (kRot) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const double x = k[i], y = k[8 + i];
                k[i] = x * cs[g][i].x - y * cs[g][i].y;
                k[8 + i] = x * cs[g][i].y + y * cs[g][i].x;
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            sa[g] = fma(q[i], k[i], sa[g]);
            sb[g] = fma(q[8 + i], k[8 + i], sb[g]);
        }
    }
    double s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        s[g] = rs_slot_sum(sa[g] + sb[g]);
        if (!valid[g]) s[g] = -INFINITY;
    }
    rs_raise_max<G>(s, st);
    double p[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        // NaN-keeping clamp, as in the decode kernels (a NaN or +inf score makes the row NaN)
        const double x = s[g] - st.m;
        p[g] = valid[g] ? exp2_f64(x < -2000.0 ? -2000.0 : x) : 0.0;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        st.l += p[g];
        double v[16];
        rs_widen(r[g].vx, v);
        rs_widen(r[g].vy, v + 8);
        // a key past the row's (a clamped row) stays out: 0 * an infinite V would be NaN
        if (valid[g]) {
#pragma unroll
            for (int i = 0; i < 16; ++i) st.o[i] = fma(p[g], v[i], st.o[i]);
        }
    }
}

// Geometry of one (row, piece) pair.
struct RsItem {
    const char* kc_seg;      // cache K rows of (b, kvh)
    const char* vc_seg;      // cache V rows of (b, kvh)
    const char* kn_seg;      // new K rows of (b, kvh), token u at u * 8 * 128 elements
    const double2* cs_seg;   // cos/sin rows of (b, token)
    int64_t stride_c;        // cache row bytes
    int st, n_keys;          // first chunk key; keys
};

// Cached chunks of this piece (ci = c0, c0 + step, ... < c_end): rows as stored, in groups
// of kRsGroup chunks computed together, kRsInflight groups in flight.  rs_prefetch requests
// the first groups (before the Q operands are formed); rs_cached runs them and the rest.
constexpr int kRsGroup = 4;
// Three or four groups in flight measured no faster (config 5: 52.7 -> 51.4 / 52.2 us;
// B=64 T=16: 28.4 -> 29.4 / 31.1 us): a piece is bound by its fp64 chains, not by memory.
constexpr int kRsInflight = 2;

__device__ __forceinline__ void rs_issue_group(const RsItem& it, int ci, int c_end, int step, RsRows (&r)[kRsGroup]) {
    const int j = threadIdx.x >> 3;
#pragma unroll
    for (int g = 0; g < kRsGroup; ++g) {
        const int cc = min(ci + g * step, max(c_end - 1, 0));
        const int64_t off = static_cast<int64_t>(min(kRsKeys * cc + j, it.n_keys - 1)) * it.stride_c;
        rs_load(it.kc_seg + off, it.vc_seg + off, r[g]);
    }
}

__device__ __forceinline__ void rs_prefetch(const RsItem& it, int c0, int c_end, int step,
                                            RsRows (&r)[kRsInflight][kRsGroup]) {
#pragma unroll
    for (int h = 0; h < kRsInflight; ++h) rs_issue_group(it, c0 + h * kRsGroup * step, c_end, step, r[h]);
}

__device__ __forceinline__ void rs_cached(const RsItem& it, int c0, int c_end, int step, const double (&q)[16],
                                          RsState& st, RsRows (&r)[kRsInflight][kRsGroup]) {
    if (c0 >= c_end) return;
    const int j = threadIdx.x >> 3;
    const double2 (*no_cs)[8] = nullptr;
    for (int ci = c0;; ci += kRsInflight * kRsGroup * step) {
#pragma unroll
        for (int h = 0; h < kRsInflight; ++h) {
            const int cg = ci + h * kRsGroup * step;
            bool valid[kRsGroup];
#pragma unroll
            for (int g = 0; g < kRsGroup; ++g) valid[g] = cg + g * step < c_end && kRsKeys * (cg + g * step) + j < it.n_keys;
            rs_chunks<kRsGroup, false>(r[h], q, valid, no_cs, st);
            if (cg + kRsGroup * step >= c_end) return;
            rs_issue_group(it, cg + kRsInflight * kRsGroup * step, c_end, step, r[h]);
        }
    }
}

// Chunks holding chunk keys (ci = c0, c0 + step, ... < c_end): a key >= start is its new
// row rotated in double with the cos/sin row of its token; a key < start (a chunk that
// straddles start) is its cache row, rotated by (1, 0), which leaves it exact.  Two in
// flight, each with its cos/sin values.
__device__ __forceinline__ void rs_new(const RsItem& it, int c0, int c_end, int step, const double (&q)[16],
                                       RsState& st) {
    if (c0 >= c_end) return;
    const int j = threadIdx.x >> 3;
    RsRows r[2];
    double2 cs[2][8];
    auto issue = [&](int ci, RsRows& rr, double2 (&cc)[8]) {
        const int key = min(kRsKeys * ci + j, it.n_keys - 1);
        const int u = max(key - it.st, 0);
        const char* krow = key >= it.st ? it.kn_seg + static_cast<int64_t>(u) * (kHkv * kD * 2)
                                        : it.kc_seg + static_cast<int64_t>(key) * it.stride_c;
        rs_load(krow, it.vc_seg + static_cast<int64_t>(key) * it.stride_c, rr);
        rs_load_cs(it.cs_seg + static_cast<int64_t>(u) * kPairs, cc);
        if (key < it.st) {
#pragma unroll
            for (int i = 0; i < 8; ++i) cc[i] = make_double2(1.0, 0.0);
        }
    };
#pragma unroll
    for (int i = 0; i < 2; ++i) issue(min(c0 + i * step, c_end - 1), r[i], cs[i]);
    for (int ci = c0;; ci += 2 * step) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int cc = ci + i * step;
            const bool valid[1] = {kRsKeys * cc + j < it.n_keys};
            rs_chunks<1, true>(&r[i], q, valid, &cs[i], st);
            if (cc + step >= c_end) return;
            issue(min(cc + 2 * step, c_end - 1), r[i], cs[i]);
        }
    }
}

// First index >= lo of the sequence p, p + step, ...
__device__ __forceinline__ int rs_first(int p, int step, int lo) {
    return p >= lo ? p : p + (lo - p + step - 1) / step * step;
}

__device__ __forceinline__ void rs_rows_path(const PrefillArgs& a, uint32_t n_rows) {
    __shared__ double o_s[kRsKeys][8][16];      // per key slot, per lane group
    const int T = a.n_new;
    const int lane = threadIdx.x;
    const int c = lane & 7;
    // The plan.  Proportional (n_rows <= 64): lane r holds row r, its pieces np_l and its
    // first item first_l; items first_l .. first_l + np_l - 1 are its pieces, and its partial
    // slots have the same numbers (the items stay below gridDim.x <= kRsSlots: the piece size
    // is set for gridDim.x - n_rows pieces, and rounding up adds at most one per row).
    // Uniform otherwise: n_pieces per row, row idx at items idx * n_pieces ...
    const bool prop = n_rows <= static_cast<uint32_t>(kWave);
    uint32_t row_l = 0;
    int np_l = 0, first_l = 0;
    int64_t n_work;
    uint32_t n_pieces = 1;
    if (prop) {
        int nc = 0;
        if (lane < static_cast<int>(n_rows)) {
            row_l = a.rs_flat[lane];
            const int64_t bt = row_l / kHq;
            nc = (a.start[bt / T] + static_cast<int>(bt % T) + kRsKeys) / kRsKeys;   // ceil((start + t + 1) / 8)
        }
        const int64_t total = wave_sum_i64(nc);
        const int64_t budget = max(static_cast<int64_t>(gridDim.x) - static_cast<int64_t>(n_rows), int64_t{1});
        const int per = static_cast<int>(max((total + budget - 1) / budget, static_cast<int64_t>(kRsMinChunks)));
        np_l = lane < static_cast<int>(n_rows) ? min(max((nc + per - 1) / per, 1), kRsMaxPieces) : 0;
        const int incl = static_cast<int>(wave_incl_scan_i64(np_l, lane));
        first_l = incl - np_l;
        n_work = __shfl(incl, kWave - 1);
    } else {
        n_pieces = gridDim.x / n_rows;      // gridDim.x <= kRsSlots
        n_pieces = n_pieces < 1 ? 1 : n_pieces > kRsMaxPieces ? kRsMaxPieces : n_pieces;
        n_work = static_cast<int64_t>(n_rows) * n_pieces;
    }
    for (int64_t wk = blockIdx.x; wk < n_work; wk += gridDim.x) {
        uint32_t idx, row;
        int piece, np;
        int64_t slot0;
        if (prop) {
            const uint64_t m = __ballot(lane < static_cast<int>(n_rows) && first_l <= wk);
            const int r = 63 - __clzll(static_cast<long long>(m));
            idx = static_cast<uint32_t>(r);
            row = __shfl(row_l, r);
            slot0 = __shfl(first_l, r);
            np = __shfl(np_l, r);
            piece = static_cast<int>(wk - slot0);
        } else {
            idx = static_cast<uint32_t>(wk / n_pieces);
            piece = static_cast<int>(wk % n_pieces);
            np = static_cast<int>(n_pieces);
            slot0 = static_cast<int64_t>(idx) * n_pieces;
            row = a.rs_flat[idx];
        }
        const int h = static_cast<int>(row % kHq);
        const int64_t bt = row / kHq;
        const int b = static_cast<int>(bt / T);
        const int t = static_cast<int>(bt % T);
        const int kvh = h / kGroup;
        RsItem it;
        it.st = a.start[b];
        it.n_keys = it.st + t + 1;
        it.stride_c = a.kv_pos_stride * 2;
        const int64_t head_elem = static_cast<int64_t>(b) * a.kv_batch_stride + static_cast<int64_t>(kvh) * a.kv_head_stride;
        it.kc_seg = reinterpret_cast<const char*>(a.k + head_elem);
        it.vc_seg = reinterpret_cast<const char*>(a.v + head_elem);
        it.kn_seg = reinterpret_cast<const char*>(a.k_new + (static_cast<int64_t>(b) * T * kHkv + kvh) * kD);
        it.cs_seg = a.rs_cs + static_cast<int64_t>(b) * T * kPairs;
        const int n_chunks = (it.n_keys + kRsKeys - 1) / kRsKeys;
        // first chunk holding a chunk key (with RoPE on K those are rotated from the new rows)
        const int c_split = (a.flags & 2u) ? it.st / kRsKeys : n_chunks;

        // Q of head h at token t, rotated at start + t (the cos/sin row of token t) and
        // scaled by scale * log2(e): this lane's 8 pairs.  Its loads are issued first, then
        // the first cached chunks', so the Q operands are formed while those are in flight.
        double q[16];
        RsRows pre[kRsInflight][kRsGroup];
        {
            const char* qrow = reinterpret_cast<const char*>(a.q + (bt * kHq + h) * kD);
            const uint4 qx = load_stream16(qrow + 16 * c);
            const uint4 qy = load_stream16(qrow + 2 * kPairs + 16 * c);
            double2 cs[8];
            rs_load_cs(a.rs_cs + bt * kPairs, cs);
            rs_prefetch(it, piece, c_split, np, pre);
            rs_widen(qx, q);
            rs_widen(qy, q + 8);
            if (a.flags & 1u) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const double x = q[i], y = q[8 + i];
                    q[i] = x * cs[i].x - y * cs[i].y;
                    q[8 + i] = x * cs[i].y + y * cs[i].x;
                }
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) q[i] *= a.qk_scale_log2;
        }

        RsState stt;
#pragma unroll
        for (int i = 0; i < 16; ++i) stt.o[i] = 0.0;
        stt.l = 0.0;
        stt.m = -INFINITY;
        rs_cached(it, piece, c_split, np, q, stt, pre);
        rs_new(it, rs_first(piece, np, c_split), n_chunks, np, q, stt);

        // The piece's O over its 8 key slots (through LDS, summed in slot order) and l.
#pragma unroll
        for (int i = 0; i < 16; ++i) o_s[lane >> 3][c][i] = stt.o[i];
        double l_tot = stt.l;
#pragma unroll
        for (int sh = 1; sh < kWave; sh <<= 1) l_tot += __shfl_xor(l_tot, sh);
        l_tot *= 0.125;                              // each key counted in its eight lanes
        __syncthreads();
        // lane i merges dims 2i, 2i + 1 (lane group cd, index ii within its 16)
        const int d0 = 2 * lane;
        const int cd = (d0 % kPairs) / 8;
        const int ii = d0 % 8 + (d0 >= kPairs ? 8 : 0);
        double o0 = 0.0, o1 = 0.0;
#pragma unroll
        for (int jj = 0; jj < kRsKeys; ++jj) {
            o0 += o_s[jj][cd][ii];
            o1 += o_s[jj][cd][ii + 1];
        }
        uint32_t* orow = reinterpret_cast<uint32_t*>(a.out + static_cast<int64_t>(row) * kD);
        if (np == 1) {
            orow[lane] = f32_to_bf16_out(static_cast<float>(o0 / l_tot)) |
                         (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(o1 / l_tot))) << 16);
        } else {
            const int64_t slot = slot0 + piece;
            unsigned long long* po = reinterpret_cast<unsigned long long*>(a.rs_part_o + slot * kD) + 2 * lane;
            store_agent(po, o0);
            store_agent(po + 1, o1);
            if (lane == 0) {
                unsigned long long* pml = reinterpret_cast<unsigned long long*>(a.rs_part_ml + slot);
                store_agent(pml, stt.m);
                store_agent(pml + 1, l_tot);
            }
            wait_vmem();                              // the stores have completed ...
            __atomic_signal_fence(__ATOMIC_SEQ_CST);  // ... and stay before the count
            int last = 0;
            if (lane == 0) last = atomicAdd(&a.rs_done[row], 1u) == static_cast<uint32_t>(np) - 1u;
            last = __shfl(last, 0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the merge's loads stay after it
            if (last) {
                // Lane u reads piece u's (m, l); lane i merges dims 2i, 2i + 1, the pieces in
                // order, kRsMergeBatch at a time: every load of a batch is issued before any
                // is used (unused entries repeat the last piece), so a batch waits for memory
                // once.  A piece with no key has m = -inf, weight 0.
                const double2 ml = load_agent_d2(reinterpret_cast<const double*>(a.rs_part_ml + slot0 + min(lane, np - 1)));
                double m_all = ml.x;
#pragma unroll
                for (int sh = 1; sh < kWave; sh <<= 1) m_all = fmax(m_all, __shfl_xor(m_all, sh));
                const int my_ex = ml.x == -INFINITY ? -1100 : max_shift_f64(ml.x, m_all);
                double lw = lane < np ? ldexp(ml.y, my_ex) : 0.0;
#pragma unroll
                for (int sh = 1; sh < kWave; sh <<= 1) lw += __shfl_xor(lw, sh);
                o0 = 0.0;
                o1 = 0.0;
                for (int u0 = 0; u0 < np; u0 += kRsMergeBatch) {
                    double2 ov[kRsMergeBatch];
#pragma unroll
                    for (int u = 0; u < kRsMergeBatch; ++u)
                        ov[u] = load_agent_d2(a.rs_part_o + (slot0 + min(u0 + u, np - 1)) * kD + 2 * lane);
#pragma unroll
                    for (int u = 0; u < kRsMergeBatch; ++u) {
                        const int ex = __shfl(my_ex, u0 + u);
                        if (u0 + u < np) {
                            o0 += ldexp(ov[u].x, ex);
                            o1 += ldexp(ov[u].y, ex);
                        }
                    }
                }
                orow[lane] = f32_to_bf16_out(static_cast<float>(o0 / lw)) |
                             (static_cast<uint32_t>(f32_to_bf16_out(static_cast<float>(o1 / lw))) << 16);
            }
        }
        __syncthreads();                // o_s is rewritten by the next work item
    }
}


// Tiles path (the flagged rows of a pair numerous enough to fill the four columns):
constexpr int kRsMinPieceKeys = 128;

// Where (tile, piece) pair wk lies: the tile's (sequence * 8 + KV head), its index j among
// that pair's tiles and the pair's flagged-row count.  Tiles are numbered pair by pair.
__device__ __forceinline__ void rs_locate(const PrefillArgs& a, int64_t ti, uint32_t per_bh, int& bh, int& j,
                                          uint32_t& cnt) {
    const int lane = threadIdx.x & (kWave - 1);
    const int n_bh = a.batch * kHkv;
    int64_t before = 0;
    bh = 0;
    j = 0;
    cnt = 0u;
    for (int base = 0; base < n_bh; base += kWave) {
        const int x = base + lane;
        const uint32_t c = x < n_bh ? min(a.rs_gcnt[x], per_bh) : 0u;
        const int64_t t = (c + 3u) / 4u;
        const int64_t incl = wave_incl_scan_i64(t, lane) + before;
        const uint64_t m = __ballot(t > 0 && incl - t <= ti && ti < incl);
        if (m) {
            const int l = __ffsll(static_cast<unsigned long long>(m)) - 1;
            bh = base + l;
            j = static_cast<int>(ti - __shfl(incl - t, l));
            cnt = __shfl(c, l);
            return;
        }
        before = __shfl(incl, kWave - 1);
    }
}

// This lane's Q operands for its column: Q row `row` (b, t, h), rotated at start + t with the
// (cos, sin) table and scaled by scale*log2(e) in double -- q[kb][e] = Q[32kb + 8(l/16) + e].
__device__ __forceinline__ void rs_q_operands(const PrefillArgs& a, uint32_t row, QOps& qa) {
    const int g = (threadIdx.x & (kWave - 1)) >> 4;
    const int64_t bt = row / kHq;
    const uint16_t* qrow = a.q + static_cast<int64_t>(row) * kD;
    const double2* cs = a.rs_cs + bt * kPairs;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        float xf[8], yf[8];
        unpack8(*reinterpret_cast<const uint4*>(qrow + 32 * kb + 8 * g), xf);
        unpack8(*reinterpret_cast<const uint4*>(qrow + kPairs + 32 * kb + 8 * g), yf);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            double x = xf[e], y = yf[e];
            if (a.flags & 1u) {
                const double2 c = cs[32 * kb + 8 * g + e];
                const double xr = x * c.x - y * c.y;
                y = x * c.y + y * c.x;
                x = xr;
            }
            qa.q[kb][e] = x * a.qk_scale_log2;
            qa.q[kb + 2][e] = y * a.qk_scale_log2;
        }
    }
}

// One 16-key chunk [kc, kc + 16) of a tile: scores of the 4 columns, each column's keys up
// to col_lim (and below k_hi) counting, online softmax and weighted V, all in fp64 (the
// arithmetic of compute_chunk).  With RoPE on K, a key >= st is its new row (loaded by the
// caller) rotated in double with the (cos, sin) row of its token.
__device__ __forceinline__ void rs_tile_chunk(const PrefillArgs& a, int b, int st, int kc, int k_hi, int col_lim,
                                              const Chunk& c, const QOps& qa, PieceState& ps) {
    __shared__ double p_lds[kWave];
    const int lane = threadIdx.x & (kWave - 1);
    double kd[4][8];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        float kf[8];
        unpack8(c.kw[kb], kf);
#pragma unroll
        for (int e = 0; e < 8; ++e) kd[kb][e] = static_cast<double>(kf[e]);
    }
    if ((a.flags & 2u) && kc + 15 >= st) {
        const int key = min(kc + (lane & 15), k_hi - 1);
        if (key >= st) {
            const int g = lane >> 4;
            const double2* cs = a.rs_cs + (static_cast<int64_t>(b) * a.n_new + (key - st)) * kPairs;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const double2 r = cs[32 * kb + 8 * g + e];
                    const double x = kd[kb][e], y = kd[kb + 2][e];
                    kd[kb][e] = x * r.x - y * r.y;
                    kd[kb + 2][e] = x * r.y + y * r.x;
                }
        }
    }
    double s4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) s4[kb] = mfma_f64(kd[kb][e], qa.q[kb][e], s4[kb]);
    const int key = kc + chunk_key_of_lane(lane);
    double s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    if (key >= k_hi || key > col_lim) s = -INFINITY;
    if (__ballot(s > ps.m_run + kMaxHeadroom)) {
        double cm = s;
        cm = fmax(cm, dpp_d<0x124>(cm));
        cm = fmax(cm, dpp_d<0x128>(cm));
        cm = swap_max_f64<true>(swap_max_f64<false>(cm));
        const bool grow = cm > ps.m_run + kMaxHeadroom;
        const double m_new = grow ? ceil(cm) : ps.m_run;
        const int shift = (ps.m_run == -INFINITY) ? 0 : max_shift_f64(ps.m_run, m_new);
        ps.l_run = ldexp(ps.l_run, shift);
#pragma unroll
        for (int i = 0; i < 8; ++i) ps.acc[i] = ldexp(ps.acc[i], shift);
        ps.m_run = m_new;
    }
    const double xs = s - ps.m_run;      // NaN-keeping clamp, as in the decode kernels
    const double p = s == -INFINITY ? 0.0 : exp2_f64(xs < -2000.0 ? -2000.0 : xs);
    ps.l_run += p;
    p_lds[(lane >> 4) * 16 + (lane & 3) * 4 + ((lane >> 2) & 3)] = p;
    const double2 pa = *reinterpret_cast<const double2*>(p_lds + (lane >> 4) * 16 + (lane & 3) * 4);
    const double2 pb = *reinterpret_cast<const double2*>(p_lds + (lane >> 4) * 16 + (lane & 3) * 4 + 2);
    const double pq[4] = {pa.x, pa.y, pb.x, pb.y};
    double vd[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float vf[8];
        unpack8(c.vw[q], vf);
#pragma unroll
        for (int e = 0; e < 8; ++e) vd[q][e] = static_cast<double>(vf[e]);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) ps.acc[e] = mfma_f64(vd[q][e], pq[q], ps.acc[e]);
}

// One BF16 output row segment: this lane's 8 dims of its column's row, O / l rounded
// double -> f32 -> BF16.
__device__ __forceinline__ void rs_write8(const PrefillArgs& a, uint32_t row, int d0, const double (&o)[8], double l) {
    uint16_t o8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o8[e] = f32_to_bf16_out(static_cast<float>(o[e] / l));
    *reinterpret_cast<bf16x8_t*>(a.out + static_cast<int64_t>(row) * kD + d0) = pack8(o8);
}

__device__ __forceinline__ void rs_tiles_path(const PrefillArgs& a, int64_t n_tiles) {
    const int T = a.n_new;
    const int lane = threadIdx.x;
    const uint32_t per_bh = 4u * static_cast<uint32_t>(T);
    int np = n_tiles >= kRsSlots ? 1 : static_cast<int>(kRsSlots / n_tiles);
    np = min(np, kRsMaxPieces);
    np = max(1, min(np, a.capacity / kRsMinPieceKeys));
    const int64_t n_work = n_tiles * np;
    const int col = lane & 3;
    const int64_t rb = a.kv_pos_stride * 2;      // cache row bytes
    for (int64_t wk = blockIdx.x; wk < n_work; wk += gridDim.x) {
        const int64_t ti = wk / np;
        const int piece = static_cast<int>(wk % np);
        int bh, j;
        uint32_t cnt;
        rs_locate(a, ti, per_bh, bh, j, cnt);
        const int b = bh / kHkv;
        const int kvh = bh % kHkv;
        const int st = a.start[b];
        const int nr = min(4, static_cast<int>(cnt) - 4 * j);
        const uint32_t* rows = a.rs_rows + static_cast<int64_t>(bh) * per_bh + 4 * j;
        // This lane's column: row `row` (a repeat of the tile's first row past nr, which
        // counts no key and is not written).
        const uint32_t row = rows[col < nr ? col : 0];
        const int col_lim = col < nr ? st + static_cast<int>((row / kHq) % T) : -1;
        int lim_max = col_lim;
        lim_max = max(lim_max, __shfl_xor(lim_max, 1));
        lim_max = max(lim_max, __shfl_xor(lim_max, 2));
        const int k_hi = lim_max + 1;                     // keys [0, k_hi) of the tile
        const int k_lo = piece * kChunk;                  // first chunk of this piece
        const int k_step = np * kChunk;

        QOps qa;
        rs_q_operands(a, row, qa);
        PieceState ps;
        init_piece(ps);
        if (k_lo < k_hi) {
            const char* kseg = reinterpret_cast<const char*>(a.k + static_cast<int64_t>(b) * a.kv_batch_stride +
                                                             static_cast<int64_t>(kvh) * a.kv_head_stride);
            const char* vseg = reinterpret_cast<const char*>(a.v + static_cast<int64_t>(b) * a.kv_batch_stride +
                                                             static_cast<int64_t>(kvh) * a.kv_head_stride);
            const bool rope_k = (a.flags & 2u) != 0;
            // Rows of chunk [kc, kc + 16): clamped to the piece's last key (masked there).  Plain
            // (cached) loads: the tiles of one pair run at the same time and read the same rows
            // (config 5 with Q x 16: 171 -> 161 us).
            auto load = [&](int kc, Chunk& c) {
                const int kk = min(kc + (lane & 15), k_hi - 1);
                const char* kp = rope_k && kk >= st
                                     ? reinterpret_cast<const char*>(
                                           a.k_new + ((static_cast<int64_t>(b) * T + (kk - st)) * kHkv + kvh) * kD)
                                     : kseg + kk * rb;
                kp += 16 * (lane >> 4);
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) c.kw[kb] = *reinterpret_cast<const uint4*>(kp + 64 * kb);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int kv = min(kc + 4 * q + (lane >> 4), k_hi - 1);
                    c.vw[q] = *reinterpret_cast<const uint4*>(vseg + kv * rb + 16 * (lane & 15));
                }
            };
            Chunk c0, c1, c2;
            load(k_lo, c0);
            load(min(k_lo + k_step, k_hi - 1), c1);
            for (int kc = k_lo; kc < k_hi; kc += k_step) {
                load(min(kc + 2 * k_step, k_hi - 1), c2);
                rs_tile_chunk(a, b, st, kc, k_hi, col_lim, c0, qa, ps);
                c0 = c1;
                c1 = c2;
            }
        }
        double l_tot;
        finish_piece(ps, l_tot);
        if (np == 1) {
            if (col < nr) rs_write8(a, row, out_dim_of_lane(lane), ps.acc, l_tot);
            continue;
        }
        // Partial at slot wk: O[column][dim] and (m, l) per column.
        {
            unsigned long long* po = reinterpret_cast<unsigned long long*>(a.rs_part_o + wk * kGroup * kD) +
                                     col * kD + out_dim_of_lane(lane);
#pragma unroll
            for (int e = 0; e < 8; ++e) store_agent(po + e, ps.acc[e]);
            if (lane < kGroup) {
                unsigned long long* pml = reinterpret_cast<unsigned long long*>(a.rs_part_ml + wk * kGroup + lane);
                store_agent(pml, ps.m_run);
                store_agent(pml + 1, l_tot);
            }
        }
        wait_vmem();                              // the stores have completed ...
        __atomic_signal_fence(__ATOMIC_SEQ_CST);  // ... and stay before the count
        int last = 0;
        if (lane == 0) last = atomicAdd(&a.rs_done[ti], 1u) == static_cast<uint32_t>(np) - 1u;
        last = __shfl(last, 0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the merge's loads stay after it
        if (!last) continue;
        // Merge: lane u reads piece u's (m, l) of all four columns; lane l then takes column
        // c = l / 16, dims 8 (l % 16) .. +7, the pieces in order, eight at a time (their loads
        // issued before any is used).  A piece with no key has m = -inf, weight 0.
        const int mc = lane >> 4;
        const int d0 = 8 * (lane & 15);
        const int64_t slot0 = ti * np;
        int ex[kGroup];
        double lw = 0.0;
        {
            double2 ml[kGroup];
#pragma unroll
            for (int c = 0; c < kGroup; ++c)
                ml[c] = load_agent_d2(
                    reinterpret_cast<const double*>(a.rs_part_ml + (slot0 + min(lane, np - 1)) * kGroup + c));
#pragma unroll
            for (int c = 0; c < kGroup; ++c) {
                double m_all = lane < np ? ml[c].x : -INFINITY;
#pragma unroll
                for (int sh = 1; sh < kWave; sh <<= 1) m_all = fmax(m_all, __shfl_xor(m_all, sh));
                ex[c] = ml[c].x == -INFINITY ? -1100 : max_shift_f64(ml[c].x, m_all);
                double lc = lane < np ? ldexp(ml[c].y, ex[c]) : 0.0;
#pragma unroll
                for (int sh = 1; sh < kWave; sh <<= 1) lc += __shfl_xor(lc, sh);
                if (c == mc) lw = lc;
            }
        }
        double o[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
        constexpr int kMb = 8;
        for (int u0 = 0; u0 < np; u0 += kMb) {
            double2 v[kMb][4];
#pragma unroll
            for (int u = 0; u < kMb; ++u) {
                const double* src = a.rs_part_o + ((slot0 + min(u0 + u, np - 1)) * kGroup + mc) * kD + d0;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[u][e] = load_agent_d2(src + 2 * e);
            }
#pragma unroll
            for (int u = 0; u < kMb; ++u) {
                int e_u = __shfl(ex[0], u0 + u);
#pragma unroll
                for (int c = 1; c < kGroup; ++c) {
                    const int x = __shfl(ex[c], u0 + u);
                    e_u = c == mc ? x : e_u;
                }
                if (u0 + u < np) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        o[2 * e] += ldexp(v[u][e].x, e_u);
                        o[2 * e + 1] += ldexp(v[u][e].y, e_u);
                    }
                }
            }
        }
        const uint32_t mrow = rows[mc < nr ? mc : 0];
        if (mc < nr) rs_write8(a, mrow, d0, o, lw);
    }
}

// The two paths share the partial slots and piece counters (a call runs one).  The tiles
// path when the flagged rows average at least kRsTileFill per (sequence, KV head) pair that
// has any: a tile of four rows costs about what one row costs on the rows path, a tile of
// one row about twice as much.
constexpr int kRsTileFill = 3;

__global__ __launch_bounds__(kWave) void rescore_kernel(PrefillArgs a) {
    const uint32_t cap = static_cast<uint32_t>(a.batch) * static_cast<uint32_t>(a.n_new) * kHq;
    const uint32_t n_rows = min(a.rs_hdr[0], cap);
    if (n_rows == 0) return;
    const uint32_t n_pairs = a.rs_hdr[1];
    if (a.rs_hdr[2] != 0u || static_cast<uint64_t>(n_rows) < static_cast<uint64_t>(kRsTileFill) * n_pairs) {
        rs_rows_path(a, n_rows);
        return;
    }
    const int lane = threadIdx.x;
    const int n_bh = a.batch * kHkv;
    const uint32_t per_bh = 4u * static_cast<uint32_t>(a.n_new);
    int64_t n_tiles = 0;
    for (int base = 0; base < n_bh; base += kWave) {
        const int x = base + lane;
        const uint32_t c = x < n_bh ? min(a.rs_gcnt[x], per_bh) : 0u;
        n_tiles += wave_sum_i64((c + 3u) / 4u);
    }
    rs_tiles_path(a, n_tiles);
}

hipError_t launch_rescore(const PrefillArgs& a, hipStream_t stream) {
    if (!a.rs_hdr) return hipSuccess;
    hipLaunchKernelGGL(rescore_kernel, dim3(static_cast<unsigned>(a.rs_wgs)), dim3(kWave), 0, stream, a);
    return hipGetLastError();
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
    const bool rq = (a.flags & 1u) != 0, rk = (a.flags & 2u) != 0;
    // Records the call's events from `from` on: a failed launch leaves none unrecorded, so
    // that the profiler can still read the call's stage times.
    auto done = [&](int from, hipError_t err) {
        if (ev)
            for (int j = from; j < kProfileEvents; ++j) (void)hipEventRecord(ev[j], stream);
        return err;
    };
    if (a.pieces_cap > 0 && !a.block_table) {
        // Single launch (small batches, contiguous cache).
        if (ev) (void)hipEventRecord(ev[0], stream);
        const dim3 grid(a.pieces_cap, batch * kHkv);
        if (rq && rk)
            hipLaunchKernelGGL((decode_single_kernel<true, true>), grid, dim3(kSingleWaves * kWave), 0, stream, a);
        else if (rq)
            hipLaunchKernelGGL((decode_single_kernel<true, false>), grid, dim3(kSingleWaves * kWave), 0, stream, a);
        else if (rk)
            hipLaunchKernelGGL((decode_single_kernel<false, true>), grid, dim3(kSingleWaves * kWave), 0, stream, a);
        else
            hipLaunchKernelGGL((decode_single_kernel<false, false>), grid, dim3(kSingleWaves * kWave), 0, stream, a);
        return done(1, hipGetLastError());
    }
    if (rq)
        hipLaunchKernelGGL((decode_prepare_kernel<true>), dim3(kHkv, batch + 1), dim3(kWave), 0, stream, a);
    else
        hipLaunchKernelGGL((decode_prepare_kernel<false>), dim3(kHkv, batch + 1), dim3(kWave), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return done(0, e);
    if (ev) (void)hipEventRecord(ev[0], stream);
    if (a.block_table) {
        if (rk)
            hipLaunchKernelGGL((decode_paged_stream_kernel<true>), dim3(a.n_wgs), dim3(kWave), 0, stream, a);
        else
            hipLaunchKernelGGL((decode_paged_stream_kernel<false>), dim3(a.n_wgs), dim3(kWave), 0, stream, a);
    } else if (rk) {
        hipLaunchKernelGGL((decode_stream_kernel<true>), dim3(a.n_wgs), dim3(kWave), 0, stream, a);
    } else {
        hipLaunchKernelGGL((decode_stream_kernel<false>), dim3(a.n_wgs), dim3(kWave), 0, stream, a);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return done(1, e);
    if (ev) (void)hipEventRecord(ev[1], stream);
    hipLaunchKernelGGL(decode_merge_kernel, dim3(kHkv, batch), dim3(kGroup * kWave), 0, stream, a);
    return done(2, hipGetLastError());
}

}  // namespace gqa

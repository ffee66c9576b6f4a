// gqa_decode.hip -- split-KV GQA decode for gfx950.
//
// One decode step of the reference core (gqa_controller.v:140-277 loop nest,
// datapath rope_unit -> bf16_dot_product_mac -> scale_unit -> flash_softmax ->
// output_accumulator) becomes two launches:
//
//   1. decode_split_kernel: grid (split, kv_head, sequence), one wave each.  The
//      wave rotates and scales the 4 Q rows of its group once, then streams its
//      slice of K/V rows from HBM exactly once, reusing every row for the 4 Q
//      heads (gqa_kv_broadcast.v:38-59).  Scores, the running max and sum, and the
//      weighted-V accumulator stay fp32 (flash_softmax.v:233-490,
//      output_accumulator.v:244-536).  It writes an unnormalised partial
//      (O[4][128], m, l) per (sequence, kv_head, split).
//   2. decode_combine_kernel: grid (q_head, sequence); merges the splits with a
//      log-sum-exp rescale, divides by the sum (output_accumulator.v:540-686) and
//      rounds to BF16 in Q-head order (gqa_output_collector.v:32-61).
//
// Masking (gqa_attention_wrapper.v:279): key p counts iff p < seq_len and
// p <= query_position.  Work is bounded to p < n_valid = min(seq_len, qpos+1);
// rows past it are never loaded, and inside the last tile invalid keys get a
// score of -inf and a probability of exactly 0 (flash_softmax.v:319-325).
//
// Lane layout inside the wave (64 lanes = 4 rows of 16): lane = 16*r + c holds
// dims [8c, 8c+8) of key (4*it + r) of the current 64-key tile; one 16-byte load
// per lane covers four whole K (or V) rows, 1 KB per wave instruction.
#include "gqa_device.h"
#include "gqa_internal.h"

namespace gqa {

constexpr int kTile = 64;             // keys per softmax tile (one per lane in phase B)
constexpr int kIters = kTile / 4;     // 4 keys per wave instruction

template <bool kRopeQ, bool kRopeK>
__global__ __launch_bounds__(kWave) void decode_split_kernel(DecodeArgs a) {
    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x;
    const int r = lane >> 4;
    const int c = lane & 15;

    const int seq_len = a.seq_len[b];
    const int qpos = a.query_pos[b];
    if (seq_len < 1 || seq_len > a.capacity || qpos < 0 || qpos >= seq_len) return;
    const int n_valid = min(seq_len, qpos + 1);
    const int k0 = split * a.split_keys;
    if (k0 >= n_valid) return;
    const int k1 = min(k0 + a.split_keys, n_valid);

    __shared__ float q_s[kGroup][kD];
    __shared__ float4 tile_s[kTile];

    // ---- Q rows of this group: RoPE at qpos in double, scale * log2(e) folded in.
    {
        const double inv_freq = a.rope.inv_freq[lane];
        double sn = 0.0, cs = 1.0;
        if (kRopeQ) sincos(static_cast<double>(qpos) * inv_freq, &sn, &cs);
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
            q_s[h][lane] = static_cast<float>(xr) * a.qk_scale_log2;
            q_s[h][lane + kPairs] = static_cast<float>(yr) * a.qk_scale_log2;
        }
    }
    __syncthreads();
    float q[kGroup][8];
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) q[h][j] = q_s[h][8 * c + j];

    const int64_t head_off = static_cast<int64_t>(b) * a.kv_batch_stride +
                             static_cast<int64_t>(kvh) * a.kv_head_stride;
    const uint16_t* kbase = a.k + head_off + 8 * c;
    const uint16_t* vbase = a.v + head_off + 8 * c;
    const int64_t ps = a.kv_pos_stride;

    float acc[kGroup][8];
    float m[kGroup], lsum[kGroup];
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        m[h] = -INFINITY;
        lsum[h] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = 0.f;
    }

    for (int t0 = k0; t0 < k1; t0 += kTile) {
        // ---- phase A: scores of 64 keys, 4 per iteration.
#pragma unroll 4
        for (int it = 0; it < kIters; ++it) {
            const int key = t0 + 4 * it + r;
            uint4 kw = make_uint4(0, 0, 0, 0);
            if (key < k1) kw = *reinterpret_cast<const uint4*>(kbase + key * ps);
            float kf[8];
            unpack8(kw, kf);
            if (kRopeK) {
                // Pair (i, i+64) sits in lanes c and c^8 of the same row.
                float other[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) other[j] = dpp_f<0x128>(kf[j]);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int i = 8 * (c & 7) + j;
                    const double x = (c < 8) ? kf[j] : other[j];
                    const double y = (c < 8) ? other[j] : kf[j];
                    double xr, yr;
                    rope_pair(x, y, key, a.rope.inv_freq[i], xr, yr);
                    kf[j] = static_cast<float>((c < 8) ? xr : yr);
                }
            }
            float s[kGroup];
#pragma unroll
            for (int h = 0; h < kGroup; ++h) {
                float t = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) t = fmaf(q[h][j], kf[j], t);
                s[h] = row16_sum(t);
            }
            if (c == 0) tile_s[4 * it + r] = make_float4(s[0], s[1], s[2], s[3]);
        }
        __syncthreads();

        // ---- phase B: online softmax, lane = key.
        const bool valid = (t0 + lane) < k1;
        const float4 s4 = tile_s[lane];
        float s[kGroup] = {s4.x, s4.y, s4.z, s4.w};
        float p[kGroup], alpha[kGroup];
#pragma unroll
        for (int h = 0; h < kGroup; ++h) {
            const float sv = valid ? s[h] : -INFINITY;
            const float m_new = fmaxf(m[h], wave_max(sv));
            alpha[h] = exp2f(m[h] - m_new);     // m = -inf on the first tile -> 0
            p[h] = valid ? exp2f(sv - m_new) : 0.f;
            lsum[h] = lsum[h] * alpha[h] + p[h];
            m[h] = m_new;
        }
        __syncthreads();
        tile_s[lane] = make_float4(p[0], p[1], p[2], p[3]);
        __syncthreads();
#pragma unroll
        for (int h = 0; h < kGroup; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[h][j] *= alpha[h];

        // ---- phase C: weighted V.
#pragma unroll 4
        for (int it = 0; it < kIters; ++it) {
            const int key = t0 + 4 * it + r;
            uint4 vw = make_uint4(0, 0, 0, 0);
            if (key < k1) vw = *reinterpret_cast<const uint4*>(vbase + key * ps);
            float vf[8];
            unpack8(vw, vf);
            const float4 p4 = tile_s[4 * it + r];
            const float pp[kGroup] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
            for (int h = 0; h < kGroup; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[h][j] = fmaf(pp[h], vf[j], acc[h][j]);
        }
        __syncthreads();
    }

    // ---- partial (O, m, l) of this split.
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        lsum[h] = wave_sum(lsum[h]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = cross_row_sum(acc[h][j]);
    }
    const int64_t pidx = (static_cast<int64_t>(b) * kHkv + kvh) * a.n_splits + split;
    if (r == 0) {
#pragma unroll
        for (int h = 0; h < kGroup; ++h) {
            float4* dst = reinterpret_cast<float4*>(a.part_o + (pidx * kGroup + h) * kD + 8 * c);
            dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
    }
    if (lane < kGroup) {
        const float mm = lane == 0 ? m[0] : lane == 1 ? m[1] : lane == 2 ? m[2] : m[3];
        const float ll = lane == 0 ? lsum[0] : lane == 1 ? lsum[1] : lane == 2 ? lsum[2] : lsum[3];
        a.part_ml[pidx * kGroup + lane] = make_float2(mm, ll);
    }
}

// One wave per (Q head, sequence); lane handles dims 2*lane and 2*lane+1.
__global__ __launch_bounds__(kWave) void decode_combine_kernel(DecodeArgs a) {
    const int qh = blockIdx.x;
    const int b = blockIdx.y;
    const int lane = threadIdx.x;
    const int kvh = qh / kGroup;
    const int h = qh % kGroup;
    uint32_t* out = reinterpret_cast<uint32_t*>(a.out + (static_cast<int64_t>(b) * kHq + qh) * kD);

    const int seq_len = a.seq_len[b];
    const int qpos = a.query_pos[b];
    if (seq_len < 1 || seq_len > a.capacity || qpos < 0 || qpos >= seq_len) {
        out[lane] = 0x7fc07fc0u;   // NaN row marks a rejected sequence
        return;
    }
    const int n_valid = min(seq_len, qpos + 1);
    const int ns = (n_valid + a.split_keys - 1) / a.split_keys;
    const int64_t base = (static_cast<int64_t>(b) * kHkv + kvh) * a.n_splits;

    float mx = -INFINITY;
    for (int s = 0; s < ns; ++s) mx = fmaxf(mx, a.part_ml[(base + s) * kGroup + h].x);
    float l = 0.f, o0 = 0.f, o1 = 0.f;
    for (int s = 0; s < ns; ++s) {
        const float2 ml = a.part_ml[(base + s) * kGroup + h];
        const float w = exp2f(ml.x - mx);
        const float2 o = reinterpret_cast<const float2*>(a.part_o + ((base + s) * kGroup + h) * kD)[lane];
        l = fmaf(ml.y, w, l);
        o0 = fmaf(o.x, w, o0);
        o1 = fmaf(o.y, w, o1);
    }
    const uint32_t lo = f32_to_bf16_rne(o0 / l);
    const uint32_t hi = f32_to_bf16_rne(o1 / l);
    out[lane] = lo | (hi << 16);
}

hipError_t launch_decode(const DecodeArgs& a, int batch, hipStream_t stream, hipEvent_t* ev) {
    const dim3 grid_split(a.n_splits, kHkv, batch);
    const dim3 grid_combine(kHq, batch);
    const bool rq = (a.flags & 1u) != 0, rk = (a.flags & 2u) != 0;
    if (ev) (void)hipEventRecord(ev[0], stream);
    if (rq && rk)
        hipLaunchKernelGGL((decode_split_kernel<true, true>), grid_split, dim3(kWave), 0, stream, a);
    else if (rq)
        hipLaunchKernelGGL((decode_split_kernel<true, false>), grid_split, dim3(kWave), 0, stream, a);
    else if (rk)
        hipLaunchKernelGGL((decode_split_kernel<false, true>), grid_split, dim3(kWave), 0, stream, a);
    else
        hipLaunchKernelGGL((decode_split_kernel<false, false>), grid_split, dim3(kWave), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ev) (void)hipEventRecord(ev[1], stream);
    hipLaunchKernelGGL(decode_combine_kernel, grid_combine, dim3(kWave), 0, stream, a);
    e = hipGetLastError();
    if (ev) (void)hipEventRecord(ev[2], stream);
    return e;
}

}  // namespace gqa

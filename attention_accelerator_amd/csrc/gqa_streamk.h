// gqa_streamk.h -- the stream-K split shared by the decode and multi-token kernels: every
// (sequence, KV head) segment's keys laid end to end in a "stream", cut into equal ranges,
// one per persistent workgroup; the part of a segment inside a range is a "piece".
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gqa_device.h"

namespace gqa {

constexpr int kMinRangeKeys = 64;    // smallest per-workgroup range
constexpr int kRangeAlign = 16;      // ranges are whole 16-key chunks

// A wave-uniform 64-bit value made scalar (shuffle results are per-lane values to the
// compiler even when every lane holds the same one).
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t x) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) x += __shfl_xor(x, d);
    return x;
}

__device__ __forceinline__ int64_t wave_max_i64(int64_t x) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) x = max(x, static_cast<int64_t>(__shfl_xor(x, d)));
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

// Each segment's span in the stream: `lead` positions that hold no key, then its keys (0
// for a sequence with no key).  A range pays for the lead of every
// segment it starts a piece of -- about what a piece's fixed cost (row merge, output or
// partial, first requests) takes in streaming time -- so that a range crossing many
// segment starts gets fewer keys and every range takes about as long.  The lead is
// kSegLead when every segment is shorter than kLeadRanges ranges, else 0: a batch of
// segments many ranges long gains little from it and its ranges would no longer line up
// with the segments (one piece each when the lengths divide evenly).
constexpr int kSegLead = 32;
constexpr int kLeadRanges = 4;

// The first piece of a range that starts at stream position x inside sequence b's
// segments, which span [off, next): its KV head, first key (0 when x falls in a segment's
// lead), the segment's keys, and x moved to the stream position of that first key.
__device__ __forceinline__ void locate_first_piece(int64_t off, int64_t next, int lead, int64_t& x, int& kvh,
                                                   int& key, int& nv) {
    const int span = static_cast<int>((next - off) / kHkv);
    const int64_t rel = x - off;
    int k = 0;
#pragma unroll
    for (int i = 1; i < kHkv; ++i) k += rel >= static_cast<int64_t>(i) * span;
    const int u = static_cast<int>(rel - static_cast<int64_t>(k) * span);
    kvh = k;
    nv = span - lead;
    key = max(u - lead, 0);
    x = off + static_cast<int64_t>(k) * span + lead + key;
}

// XCD-weighted ranges.  Workgroups are dealt round-robin over the 8 XCDs (block w runs
// on XCD w % 8).  In a plain streaming probe on MI355X a wave on an odd XCD read about 7 %
// slower than one on an even XCD (swapping ranges between neighbours left the slowness
// with the XCD), though which XCDs lag varies between launches and kernels; the weighting
// is a per-path measured default.  Each pair of blocks (2j, 2j+1) covers 2 * per
// positions, the even block per + extra of them, the odd one per - extra.
__device__ __forceinline__ int64_t range_start(int64_t per, int64_t extra, int64_t w) {
    return (w >> 1) * 2 * per + ((w & 1) ? per + extra : 0);
}

// The range holding stream position x.
__device__ __forceinline__ int64_t range_of(int64_t per, int64_t extra, int64_t x) {
    const int64_t j = x / (2 * per);
    return 2 * j + (x - 2 * j * per >= per + extra ? 1 : 0);
}

// Positions moved from each odd range to its even neighbour: skew_pm per mille of a
// range, whole 16-key chunks.
__device__ __forceinline__ int64_t range_extra(int64_t per, int skew_pm) {
    return per * skew_pm / 1000 / kRangeAlign * kRangeAlign;
}

// Range size for `total` stream positions over n_wgs workgroups.
__device__ __forceinline__ int64_t range_size(int64_t total, int n_wgs) {
    int64_t per = (total + n_wgs - 1) / n_wgs;
    per = per < kMinRangeKeys ? kMinRangeKeys : per;
    return (per + kRangeAlign - 1) / kRangeAlign * kRangeAlign;
}

// The lead and the stream totals from the batch's keys per segment: their sum over the
// sequences, their maximum and the number of sequences with keys.
// seg_lead: the lead a path charges per segment start (kSegLead for decode).  A lead above
// kSegLead is cut to a quarter of the lead-free range size (never below kSegLead), so that
// a range always reaches past a lead into keys.
__device__ __forceinline__ void plan_lead_totals(int64_t sum, int max_keys, int n_seq, int n_wgs, int& lead,
                                                 int64_t& total, int64_t& per_wg, int seg_lead = kSegLead) {
    const int64_t per0 = range_size(sum * kHkv, n_wgs);
    int want = seg_lead;
    if (want > kSegLead) {
        const int64_t quarter = per0 / 4 / kRangeAlign * kRangeAlign;
        want = static_cast<int>(max(static_cast<int64_t>(kSegLead), min(static_cast<int64_t>(want), quarter)));
    }
    lead = static_cast<int64_t>(max_keys) < kLeadRanges * per0 ? want : 0;
    total = (sum + static_cast<int64_t>(n_seq) * lead) * kHkv;
    per_wg = range_size(total, n_wgs);
}

}  // namespace gqa

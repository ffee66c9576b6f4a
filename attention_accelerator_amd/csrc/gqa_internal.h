// gqa_internal.h -- kernel argument blocks and launchers behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gqa.h"
#include "gqa_device.h"

namespace gqa {

// Everything one decode launch needs, passed by value as the kernel argument.
struct DecodeArgs {
    const uint16_t* q;        // [B][32][128]
    const uint16_t* k;        // rows at b*kv_batch_stride + h*kv_head_stride + p*kv_pos_stride
    const uint16_t* v;
    const int32_t* seq_len;   // [B]
    const int32_t* query_pos; // [B]
    uint16_t* out;            // [B][32][128]
    double* q_op;             // [B][8][4][128] Q rows rotated at query_pos and scaled by scale*log2(e)
    int64_t* plan_hdr;        // {total keys, keys per stream workgroup}
    int64_t* seq_off;         // [B+1] first global key offset of sequence b's segments
    int32_t* seq_nreal;       // [B] keys of sequence b that count (n_valid; the plan pads to blocks)
    double* part_o;           // [n_slots][4][128] unnormalised partial outputs
    double2* part_ml;         // [n_slots][4] (integer-valued running max in log2 units, sum)
    unsigned long long* seg_count;  // [B*8] pieces finished per segment, single-launch path (zero between calls)
    const int32_t* block_table;  // paged cache: [B][max_blocks] block ids (nullptr: contiguous cache)
    int64_t kv_batch_stride;  // contiguous: elements per sequence; paged: per block of the pool
    int64_t kv_head_stride;
    int64_t kv_pos_stride;
    int32_t capacity;         // positions per sequence (paged: max_blocks * 16)
    int32_t max_blocks;       // paged: block-table entries per sequence
    int32_t n_blocks;         // paged: blocks in the pool (ids outside [0, n_blocks) poison the row)
    int32_t batch;
    int32_t n_wgs;            // persistent workgroups of the stream kernel
    int32_t skew_pm;          // stream and paged kernels: XCD weighting of the ranges (per mille)
    int32_t pieces_cap;       // > 0: single-launch path, pieces per segment (grid x)
    int32_t piece_keys;       // single-launch path: keys per piece
    double qk_scale_log2;     // scale * log2(e), folded into Q
    uint32_t flags;           // bit0 RoPE on Q, bit1 RoPE on K
    RopeTable rope;
};

// Launch plan for a batch: stream-kernel workgroups and partial slots, or (small batches)
// the single-launch piece size.
struct DecodePlan {
    int32_t n_wgs;
    int32_t pieces_cap;       // > 0 selects the single-launch path
    int32_t piece_keys;
    int64_t n_slots;          // stream path: n_wgs + 8 * batch; single path: 8 * batch * pieces_cap
    size_t part_o_bytes;      // fp64 partial outputs at offset 0
    size_t part_ml_bytes;     // then the (m, l) pairs
    size_t q_op_bytes;        // then the prepared Q operands
    size_t plan_bytes;        // then the plan: header, seq_off[B+1], seq_nreal[B]
    size_t count_bytes;       // then the per-segment counters of the single-launch path
    size_t workspace_bytes;
};

// max_single_segments >= 0 caps the segments (batch * 8) a single-launch plan may count in
// (its per-segment counters); larger batches take the stream path.  The plan follows the
// arguments and the device only (params: stream_wgs and the GQA_PLAN_* flags).
DecodePlan plan_decode(const gqa_params_t* params, int32_t batch, int32_t capacity, bool paged = false,
                       int64_t max_single_segments = -1);
// Largest gqa_params_t.stream_wgs accepted.
constexpr int32_t kStreamWgsMax = 65536;
// ev (optional): three events recorded before the split kernel, between the two
// kernels and after the combine kernel.
hipError_t launch_decode(const DecodeArgs& a, int batch, hipStream_t stream,
                         hipEvent_t* ev = nullptr);
hipError_t launch_zero_words(uint32_t* p, int64_t n, hipStream_t stream);

struct RopeArgs {
    const uint16_t* in;
    uint16_t* out;
    const int32_t* positions;
    int64_t n_rows;
    int64_t row_stride;
    int32_t pos0;
    RopeTable rope;
};

hipError_t launch_rope_rows(const RopeArgs& a, hipStream_t stream);

void fill_rope_table(double theta, RopeTable* t);

// Chunked prefill: n_new query tokens per sequence appended after start[b] cached
// positions (gqa_prefill.hip).
struct PrefillArgs {
    const uint16_t* q;        // [B][T][32][128]
    const uint16_t* k_new;    // [B][T][8][128] new K rows as given (unrotated when RoPE on K)
    const uint16_t* v_new;    // [B][T][8][128]
    uint16_t* k;              // cache, rows at b*kv_batch_stride + h*kv_head_stride + p*kv_pos_stride
    uint16_t* v;              // (paged: block_table[b][p/16]*kv_batch_stride + h*kv_head_stride
                              //  + (p%16)*kv_pos_stride)
    const int32_t* block_table;  // paged cache: [B][max_blocks] (nullptr: contiguous)
    int32_t max_blocks;
    int32_t n_blocks;
    const int32_t* start;     // [B] cached positions before the chunk (device)
    uint16_t* out;            // [B][T][32][128]
    float* kx32;              // [B][T][8][128] rotated new K rows in fp32, not rounded to BF16
                              // (nullptr: append only)
    // fp16 staging of the attention kernel's K/V (prefill_stage_kernel): per (sequence, KV
    // head, block of 64 positions) a power-of-two scale puts the block's largest magnitude
    // in [2^14, 2^15), so every BF16 value of the block converts to fp16 exactly except
    // ones more than 2^31 below that largest magnitude.
    uint16_t* stg_k;          // [B][8][stg_pos][128] fp16 K rows (chunk keys: leading part)
    uint16_t* stg_v;          // [B][8][stg_pos][128] fp16 V rows
    uint16_t* stg_klo;        // [B][8][stg_cb][64][128] fp16 trailing parts of the chunk keys of
                              // the blocks that hold them (0 for cached keys)
    uint32_t* stg_scale;      // [B][8][stg_pos / 64]: K scale exponent (int8), V scale exponent
                              // (int8) << 8, bit 31 set when the block cannot be staged exactly
    int32_t stg_pos;          // positions per (sequence, KV head): capacity rounded up to 64
    int32_t stg_cb;           // chunk blocks per (sequence, KV head): ceil(T / 64) + 1
    int64_t kv_batch_stride;
    int64_t kv_head_stride;
    int64_t kv_pos_stride;
    int32_t capacity;
    int32_t batch;
    int32_t n_new;            // T
    int32_t n_qblk;           // query blocks of 32 positions per sequence
    double qk_scale_log2;     // scale * log2(e), folded into Q
    uint32_t flags;           // bit0 RoPE on Q, bit1 RoPE on the new K rows
    RopeTable rope;
    // Multi-token path (n_new <= kMultiMaxNew): the stream-K split of the decode path, W =
    // multi_waves(n_new) column tiles of 16 (4 heads x 4 tokens) per segment.
    float4* q_op;             // [B][8][W][8][64] Q rotated and scaled, f32, in the MFMA B layout
                              // (float4 2kb + h of lane (g, n): dims 32kb + 8g + 4h .. +3)
    int64_t* plan_hdr;        // {total stream positions, positions per workgroup, segment lead,
                              //  positions moved from odd to even ranges}
    int64_t* seq_off;         // [B+1] stream position of sequence b's first segment
    float* part_o;            // [n_slots][16W][128] unnormalised partial outputs (column 16w + 4t + h)
    float2* part_ml;          // [n_slots][16W] (integer-valued running max in log2 units, sum)
    float* chunk_s;           // [B][8][16W][4W] scores of the chunk's keys u per column (log2 units)
    uint32_t* piece_st;       // [n_slots][W][8 + 128] each piece's (and wave's) cached-key maxima for
                              // the rescore flag (K pair-group norms, |V| codes), reduced by the merge
    int32_t n_wgs;            // persistent workgroups of the multi-token stream kernel
    int32_t skew_pm;          // XCD weighting of the ranges (per mille of a range)
    // fp64 rescore of the output rows the MFMA kernels may have computed outside 64 BF16 ULP
    // (the attention epilogue or the multi-token merge decides, rescore_kernel recomputes); rs_hdr
    // nullptr: off.
    uint32_t* rs_hdr;         // [2]: flagged rows, (sequence, KV head) pairs with one
    uint32_t* rs_flat;        // [B*T*32] flagged rows (b*T + t)*32 + q_head, in flagging order
    uint32_t* rs_rows;        // [B*8][4T] the same rows by (sequence, KV head)
    uint32_t* rs_gcnt;        // [B*8] flagged rows per (sequence, KV head)
    uint32_t* rs_done;        // [B*T*32] finished pieces per flagged row or tile of rows
    double2* rs_cs;           // [B][T][64] cos, sin of (start + t) * inv_freq[i] (RoPE on Q or K)
    double* rs_part_o;        // [kRsSlots][4][128] unnormalised partial outputs (a tile's rows, or
                              // one row per slot ([kRsSlots][128]) on the rows path)
    double2* rs_part_ml;      // [kRsSlots][4] (running max, sum)
    int32_t rs_wgs;           // workgroups of the rescore kernel
    // What the flag decision reads besides the output rows and Q:
    float* rs_m;              // [B*T*32] the row's running max (log2 units); NaN: always rescore
    // Over the keys of segment (b, kv head) before chunk block cb (cb = 0: the cached keys,
    // which every new token sees): the largest squared norm of each pair group (dims 8g ..
    // 8g+7 and 64+8g .. 64+8g+7, g < 8: the RoPE pairs, so a norm does not change under
    // rotation), fp32 bits, and the largest |V| of each dim, BF16 bits.  Maxima of
    // non-negative values compared as bit patterns: prefill_stat_reduce_kernel writes every
    // entry (order-independent); the multi-token merge kernel keeps its segment's in LDS.
    uint32_t* rs_kc;          // [B*8][rs_ncb][8]
    uint32_t* rs_dc;          // [B*8][rs_ncb][128]
    // The same maxima over the chunk's keys, running over the key positions: entry (cb, r)
    // covers every key up to row r of chunk block cb (prefill: the 64-position blocks that
    // hold chunk keys, r = position % 64, including the cached rows at the start of the
    // first block; multi-token: one block of T rows, r = token).  Entry (cb, rs_nr - 1) is
    // block cb's maximum.
    uint32_t* rs_kpre;        // [B*8][rs_ncb][rs_nr][8]
    uint16_t* rs_dpre;        // [B*8][rs_ncb][rs_nr][128]
    int32_t rs_ncb;
    int32_t rs_nr;
    // Prefill: the maxima of each 64-position block of cached keys (the staging kernel writes
    // them, prefill_stat_reduce_kernel folds them into rs_kc / rs_dc); |V| codes packed two
    // per dword (dims 2c, 2c + 1).
    uint32_t* rs_kblk;        // [B*8][rs_nblk][8]
    uint32_t* rs_dblk;        // [B*8][rs_nblk][64]
    int32_t rs_nblk;
};

// Rescore: an output row of the MFMA paths is recomputed in fp64 when one of its elements may
// lie within the paths' error of zero, where 64 BF16 ULP of the element is less than that
// error.  The paths' error in output dim j follows two things:
//   * the error of each score, a sum of products q_i k_i accumulated in fp32: it grows with
//     sum |q_i k_i|, which may be far above the score itself when the products cancel.
//     By Cauchy-Schwarz over the 8 pair groups G, sum |q_i k_i| <= E = scale * log2(e) *
//     sum_G |q_G| * max_k |k_G| (the max over the keys the row sees).
//   * the spread of V in dim j: a score error moves weight between keys, which changes
//     output j in proportion to dim j's V values.
// So each element is measured in units of its dim's V scale, y_j = x_j / D_j with D_j =
// max_k |v_kj| over the keys the row sees, and a row is rescored when
//     min_j |y_j| < 2^-17 * F * rms(y),   F = max(1, |m| / 6, E / 32)
// (m: the row's running max, log2 units).  For N(0,1) inputs (E ~ 23-27, |m| ~ 5-7, F = 1)
// the largest error measured on the MFMA paths, beyond the output's own BF16 rounding, is
// 1.18e-6 of the row's rms (two draws of 2.1M outputs of the prefill kernel; 8.6e-7 with
// the multi-token kernels' three BF16 parts); a 64-ULP miss needs an error of a quarter of
// the element, so an element below ~4.7e-6 rms, and 2^-17 = 7.6e-6 flags those with a
// margin of 1.6 (about 7e-4 of N(0,1) rows).  Rows whose products cancel (dims i and i+64
// of Q equal and of K opposite, x 2^6: E ~ 1.1e5 with |m| ~ 2) err about 8 times less per
// unit of E than N(0,1) rows in a CPU emulation of the kernels' fp32 accumulation order,
// and rows whose first-half products are all positive and cancel against the second half
// (the largest partial sums the 4 x 32-dim MFMA steps can carry) about 1.9 times less;
// outlier V channels (x 2^6 .. 2^14) err in proportion to their own D_j.
// Squared: 128 min y^2 <= 2^-34 F^2 sum y^2, in double.
constexpr double kRsFlagRatio2 = 1.0 / 17179869184.0;    // (2^-17)^2
constexpr double kRsFlagScore = 6.0;
constexpr double kRsFlagE = 32.0;

// The decision for one row: mn2 = smallest y_j^2 over the dims with D_j > 0, ss = sum y^2
// (both formed in double: see the callers), m = running max, e = E.  Not finite: rescored.
// A row whose every element is exactly zero while some D_j > 0 (mn2 = ss = 0) is rescored
// too; with no D_j > 0 (mn2 = inf) the row is exactly zero and is not.
__host__ __device__ inline bool rs_flag_decide(double mn2, double ss, double m, double e) {
    if (!(ss <= 1e300) || !(e <= 1e300) || !(m == m)) return true;
    double f2 = 1.0;
    const double fm = m * m * (1.0 / (kRsFlagScore * kRsFlagScore));
    const double fe = e * e * (1.0 / (kRsFlagE * kRsFlagE));
    f2 = fm > f2 ? fm : f2;
    f2 = fe > f2 ? fe : f2;
    return mn2 * kD <= kRsFlagRatio2 * f2 * ss;
}
// HIP events per call of the opt-in kernel timing: up to four stages between them.
constexpr int kProfileEvents = 5;
constexpr int kRsSlots = 1024;                            // partial slots (tiles x pieces)
constexpr int kRsMaxPieces = 64;                          // pieces per tile at most
// Rescore region of a workspace; ncb, nr: the chunk-prefix blocks and rows (prefill:
// ceil(T / 64) + 1 and 64; multi-token: 1 and T); nblk: 64-position blocks of the cache
// (prefill; 0 for multi-token).
size_t rescore_bytes(int32_t batch, int32_t n_new, int32_t ncb, int32_t nr, int32_t nblk);
void rescore_layout(PrefillArgs& a, const gqa_params_t* params, void* base, int32_t ncb, int32_t nr, int32_t nblk);
// Prefill: the cached-key maxima from the staging kernel's block maxima.
hipError_t launch_prefill_stat_reduce(const PrefillArgs& a, hipStream_t stream);
// The fp64 rescore of the flagged rows (after the kernels that decide the flags).
hipError_t launch_rescore(const PrefillArgs& a, hipStream_t stream);

// Chunk blocks of the prefill path's prefix statistics (64-position blocks holding chunk keys).
__host__ __device__ constexpr int32_t prefill_chunk_blocks(int32_t n_new) { return (n_new + 63) / 64 + 1; }
// 64-position blocks of a cache of `capacity` positions (the staging planes' blocks).
__host__ __device__ constexpr int32_t prefill_cache_blocks(int32_t capacity) { return (capacity + 63) / 64; }

// Appends a flagged output row (device side).
__device__ __forceinline__ void rs_append(const PrefillArgs& a, uint32_t row) {
    const uint32_t i = atomicAdd(a.rs_hdr, 1u);
    if (i < static_cast<uint32_t>(a.batch) * static_cast<uint32_t>(a.n_new) * kHq) a.rs_flat[i] = row;
    const uint32_t per = 4u * static_cast<uint32_t>(a.n_new);            // rows of one (b, kv head)
    const uint32_t bh = row / (static_cast<uint32_t>(a.n_new) * kHq) * kHkv + (row % kHq) / kGroup;
    const uint32_t j = atomicAdd(a.rs_gcnt + bh, 1u);
    if (j < per) a.rs_rows[bh * per + j] = row;
    if (j == 0u) atomicAdd(a.rs_hdr + 1, 1u);                          // pairs with a flagged row
}

// Clears the flagged-row count (the first kernel of a prefill or multi-token call).
// Header words: flagged rows, (sequence, KV head) pairs with one, and a nonzero word when a
// flagged row sees a V that is not finite (the rescore then takes its rows path: the tiles
// path shares V between rows of different causal limits, and 0 * inf would give NaN).
__device__ __forceinline__ void rs_clear(const PrefillArgs& a, int t) {
    if (a.rs_hdr && t < 3) a.rs_hdr[t] = 0u;
}

// The same kernel clears row (b*T + t)*32 + h's piece counter and, with RoPE on K, stores
// the cos/sin table row of token t.

// Chunks of at most this many new tokens per sequence take the multi-token path.
constexpr int32_t kMultiMaxNew = 16;
// Waves per workgroup (16-column tiles) of the multi-token path for T new tokens: 1, 2 or 4.
int32_t multi_waves(int32_t n_new);
// Waves per SIMD of that path's stream kernel: 1 for one tile, 2 for two or four tiles.
int32_t multi_simd_waves(int32_t n_new);

// Workspace of the prefill attention path (chunks of more than kMultiMaxNew tokens): the
// fp32 rotated new K rows, then the fp16 staging planes and block scales.
size_t prefill_stage_bytes(int32_t batch, int32_t n_new, int32_t capacity);
void prefill_stage_layout(PrefillArgs& a, void* base);
hipError_t launch_prefill_stage(const PrefillArgs& a, hipStream_t stream);
// Workspace of the multi-token path: Q operands, plan, partials, chunk-key scores.
size_t prefill_multi_bytes(int32_t batch, int32_t n_new, int32_t n_wgs);
void prefill_multi_layout(PrefillArgs& a, void* base, int32_t n_wgs);
hipError_t launch_kv_append(const PrefillArgs& a, hipStream_t stream);
hipError_t launch_prefill_attention(const PrefillArgs& a, hipStream_t stream);
// The multi-token path's three kernels; ev (optional): events recorded before its stream
// kernel and after it (the merge follows).
hipError_t launch_prefill_multi(const PrefillArgs& a, hipStream_t stream, hipEvent_t* ev = nullptr);


}  // namespace gqa

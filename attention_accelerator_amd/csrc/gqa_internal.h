// gqa_internal.h -- kernel argument blocks and launchers behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
// (its per-segment counters); larger batches take the stream path.
DecodePlan plan_decode(int32_t batch, int32_t capacity, bool paged = false, int64_t max_single_segments = -1);
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
    uint4* q_op;              // [B][8][W][3][4][64] Q operands (3 BF16 parts, MFMA B layout)
    int64_t* plan_hdr;        // {total stream positions, positions per workgroup, segment lead,
                              //  positions moved from odd to even ranges}
    int64_t* seq_off;         // [B+1] stream position of sequence b's first segment
    float* part_o;            // [n_slots][16W][128] unnormalised partial outputs (column 16w + 4t + h)
    float2* part_ml;          // [n_slots][16W] (integer-valued running max in log2 units, sum)
    float* chunk_s;           // [B][8][16W][4W] scores of the chunk's keys u per column (log2 units)
    int32_t n_wgs;            // persistent workgroups of the multi-token stream kernel
    int32_t skew_pm;          // XCD weighting of the ranges (per mille of a range)
    // fp64 rescore of the output rows the MFMA kernels flag (an element within
    // kRsFlagRatio of its row's rms from zero); rs_hdr nullptr: off.
    uint32_t* rs_hdr;         // [1]: flagged rows
    uint32_t* rs_rows;        // [B*T*32] flagged rows, (b*T + t)*32 + q_head, in flagging order
    uint32_t* rs_done;        // [B*T*32] finished pieces per flagged row (indexed by row)
    double2* rs_cs;           // [B][T][64] cos, sin of (start + t) * inv_freq[i] (RoPE on Q or K)
    double* rs_part_o;        // [kRsSlots][128] unnormalised partial output rows
    double2* rs_part_ml;      // [kRsSlots] (running max, sum)
    int32_t rs_wgs;           // workgroups of the rescore kernel
};

// Rescore: an output row is recomputed in fp64 when one of its elements lies closer to zero
// than kRsFlagRatio times the row's rms.  The largest error measured on the MFMA paths (the
// excess over the output's own BF16 rounding) is 8.6e-7 of the row's rms with three BF16
// parts (4.8M outputs of N(0,1) inputs) and 8.9e-7 and 1.18e-6 with the prefill kernel's two
// fp16 parts (two draws of 2.1M outputs), so a 64-BF16-ULP miss, which needs an error of a
// quarter of the element, needs an element below ~4.7e-6 of the rms; 2^-17 = 7.6e-6 flags
// those with a margin of 1.6.  Squared: min^2 * 128 < ratio^2 * sum x^2.
constexpr double kRsFlagRatio2 = 1.0 / 17179869184.0;    // (2^-17)^2
// Those errors were measured on rows whose running max m (log2 units) is at most ~6.  The
// scores are fp32 sums of the products q_i k_i, so their error scales with sum |q_i k_i|,
// which for the keys that carry a row's softmax is about twice |m| (random rows; a key far
// above the others dominates the row and its own error cancels in the normalisation).  The
// threshold therefore grows with |m| past kRsFlagScore: Q scaled by 16 (|m| ~ 85) has errors
// ~16 times those above, and without this a few of its elements missed 64 ULP unflagged.
constexpr double kRsFlagScore = 6.0;

// Whether an output row (smallest element magnitude mn, sum of squares ss, running max m in
// log2 units) goes to the fp64 rescore.  A row that is not finite always does: scores past
// the fp32 range (Q and K both far from 1, e.g. 2^100 and 2^40) make the MFMA paths' row NaN
// where the double golden is finite.
__host__ __device__ inline bool rs_flag_row(double mn, double ss, float m) {
    if (!(ss <= 1e300)) return true;
    const double mm = static_cast<double>(m) * static_cast<double>(m) * (1.0 / (kRsFlagScore * kRsFlagScore));
    return mn * mn * kD < kRsFlagRatio2 * (mm > 1.0 ? mm : 1.0) * ss;
}
constexpr int kRsSlots = 1024;                            // partial slots (rows x pieces)
constexpr int kRsMaxPieces = 64;                          // pieces per row at most (one per lane)
size_t rescore_bytes(int32_t batch, int32_t n_new);
void rescore_layout(PrefillArgs& a, void* base);
hipError_t launch_rescore(const PrefillArgs& a, hipStream_t stream);

// Appends a flagged output row (device side).
__device__ __forceinline__ void rs_append(const PrefillArgs& a, uint32_t row) {
    const uint32_t i = atomicAdd(a.rs_hdr, 1u);
    if (i < static_cast<uint32_t>(a.batch) * static_cast<uint32_t>(a.n_new) * kHq) a.rs_rows[i] = row;
}

// Clears the flagged-row count (the first kernel of a prefill or multi-token call).
__device__ __forceinline__ void rs_clear(const PrefillArgs& a, int t) {
    if (a.rs_hdr && t == 0) a.rs_hdr[0] = 0u;
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

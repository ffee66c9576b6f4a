/*
 * gqa.h -- C ABI of libgqa.so: the Llama-3-8B GQA attention step on MI355X (gfx950).
 *
 * Geometry is fixed, as in the reference core: 32 Q heads over 8 KV heads (group 4),
 * head_dim 128, BF16 in and out, RoPE rotate_half with theta 500000, scores scaled
 * by 1/sqrt(128), masked online softmax, weighted V.
 *
 * The ABI replaces the reference core's host contract:
 *   - AXI-Lite register file          axi_lite_regs.v:5-24 (N_Q_HEADS, N_KV_HEADS,
 *     HEAD_DIM, TILE_DIM, SEQ_LEN, N_KV_TILES, SCALE, QUERY_POSITION, CTRL.start,
 *     STATUS.done/error)                        -> gqa_params_t + per-sequence arrays
 *   - start-time config rejection      gqa_attention_wrapper.v:230-244
 *                                               -> gqa_validate_registers / status codes
 *   - AXIS ingress of Q rows and K/V rows in position order (README.md:24-39,
 *     tests/tb_gqa_attention_wrapper.sv:174-193)  -> device pointers + gqa_kv_layout_t
 *   - AXIS egress, 32 rows x 128 BF16 in Q-head order (gqa_output_collector.v:32-61)
 *                                               -> out[B][32][128]
 *   - rope_unit (rope_unit.v:38-330) in isolation, as tests/tb_rope_unit.sv drives it
 *                                               -> gqa_rope_rows_bf16
 *
 * Conventions: every data pointer is a device pointer; BF16 values are passed as
 * their 16-bit codes.  Calls are asynchronous on `stream` (a hipStream_t, NULL =
 * the default stream) and allocate nothing; the caller owns every buffer,
 * including the workspace.  On any non-zero status nothing was launched and no
 * output was written (the reference suppresses start and raises its error flag).
 * Calls are re-entrant from any host thread given distinct workspaces.
 */
#ifndef GQA_H
#define GQA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  GQA_ERR_INVALID_CONFIG is the STATUS.error of
 * gqa_attention_wrapper.v:288 (bad geometry, zero scale, bad lengths). */
enum gqa_status {
    GQA_OK = 0,
    GQA_ERR_INVALID_CONFIG = 1,
    GQA_ERR_BAD_POINTER = 2,   /* NULL or misaligned pointer / stride */
    GQA_ERR_WORKSPACE = 3,     /* workspace missing or smaller than required */
    GQA_ERR_HIP = 4            /* the HIP runtime refused the launch */
};

/* Operand rotation flags.  The reference rotates Q at query_position and every
 * K row at its cache position (gen_gqa_wrapper_vectors.py:124-126,
 * gqa_attention_wrapper.v:302-308).  A cache stored post-RoPE drops GQA_ROPE_K. */
#define GQA_ROPE_Q 1u
#define GQA_ROPE_K 2u

/* Plan flags (no counterpart in the reference; tests and tuning, results stay within the
 * same tolerance): GQA_PLAN_STREAM_K makes every contiguous decode call take the
 * three-launch stream-K plan (small batches otherwise run as one launch);
 * GQA_PLAN_NO_MULTI_TOKEN sends chunks of at most 16 new tokens through the prefill
 * attention kernel instead of the multi-token stream-K path.  Workspace sizes follow them. */
#define GQA_PLAN_STREAM_K 4u
#define GQA_PLAN_NO_MULTI_TOKEN 8u

/* Geometry, scale and RoPE: the register subset that shapes the arithmetic.
 * Only n_q_heads=32, n_kv_heads=8, head_dim=128 are accepted
 * (gqa_attention_wrapper.v:231-233).  Zero-initialise the struct: stream_wgs = 0 is the
 * default.  Every workspace size depends on these fields, the call's sizes and the current
 * device's CU count only (never on the environment). */
typedef struct gqa_params {
    int32_t n_q_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    double scale;         /* score scale, normally 1/sqrt(128) (the golden's double,
                             gen_gqa_wrapper_vectors.py:129); 0 is rejected (wrapper.v:237) */
    double rope_theta;    /* normally 500000; must be > 0 when a RoPE flag is set */
    uint32_t flags;       /* GQA_ROPE_Q | GQA_ROPE_K, GQA_PLAN_* */
    int32_t stream_wgs;   /* persistent workgroups of the stream-K kernels: 0 = four per CU
                             of the current device (tuning and tests: 1 .. 65536) */
} gqa_params_t;

/* Where K/V rows live.  Row (sequence b, KV head h, position p) starts at element
 * b*batch_stride + h*head_stride + p*pos_stride of the K (and V) base; each row
 * is 128 contiguous BF16.  Strides are in elements and multiples of 8; pointers
 * 16-byte aligned.  capacity = positions allocated per sequence; the rows of one
 * (sequence, KV head) must span less than 4 GiB ((capacity + 64) * pos_stride * 2
 * bytes). */
typedef struct gqa_kv_layout {
    int64_t batch_stride;
    int64_t head_stride;
    int64_t pos_stride;
    int32_t capacity;
} gqa_kv_layout_t;

/* Host-side check of the reference's register set, as the core does at start
 * (gqa_attention_wrapper.v:230-237): n_q_heads==32, n_kv_heads==8, head_dim==128,
 * tile_dim==16, seq_len!=0, n_kv_tiles==ceil(seq_len/kv_block_len), scale_bf16!=0.
 * kv_block_len is the core's KV_BLOCK_LEN parameter (16, or 4 on PYNQ-Z2).
 * Returns GQA_OK or GQA_ERR_INVALID_CONFIG. */
int gqa_validate_registers(int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           int32_t tile_dim, int32_t seq_len, int32_t n_kv_tiles,
                           int32_t kv_block_len, uint16_t scale_bf16);

/* Host-side check of per-sequence lengths (host arrays): 1 <= seq_len[b] <= capacity
 * and 0 <= query_pos[b] < seq_len[b] (gen_gqa_wrapper_vectors.py:73-78).  The
 * decode call reads its length arrays on the device; callers holding host copies
 * use this to reject bad lengths before launching.  Returns GQA_OK or
 * GQA_ERR_INVALID_CONFIG. */
int gqa_validate_lengths(const int32_t* seq_len, const int32_t* query_pos, int32_t batch,
                         int32_t capacity);

/* Workspace bytes gqa_decode_bf16 needs for `batch` sequences of up to `capacity`
 * positions.  0 if the configuration is invalid. */
size_t gqa_decode_workspace_bytes(const gqa_params_t* params, int32_t batch, int32_t capacity);

/* Zero-fill a decode workspace with a fill kernel on `stream` (no memset, so the call
 * may sit inside a captured graph).  Required once before a workspace's first decode
 * call: small batches finish in one launch and count finished pieces in it (each call
 * leaves the counters at zero again).  A workspace prepared for (batch, capacity) serves
 * later calls with the same batch and capacity only: before a call with another batch or
 * capacity, call gqa_decode_workspace_init again (the counters sit where that plan puts
 * them; stale partial data there would leave output rows unwritten).  No reference
 * counterpart. */
int gqa_decode_workspace_init(const gqa_params_t* params, int32_t batch, int32_t capacity,
                              void* workspace, size_t workspace_bytes, void* stream);

/* One decode step for a batch of sequences (the reference core computes batch 1):
 *   q          [batch][32][128]  Q rows of the token at query_pos[b]
 *   k, v       cache rows per `kv` (positions in order)
 *   seq_len    [batch] int32, device: valid cache length
 *   query_pos  [batch] int32, device: position of the query token
 *   out        [batch][32][128]  output rows in Q-head order
 *   workspace  gqa_decode_workspace_bytes bytes, prepared once by
 *              gqa_decode_workspace_init for this batch and capacity; calls sharing a
 *              workspace must be ordered (same stream)
 * Batches whose caches hold at most 2^18 keys in all (batch * 8 * capacity) run as one
 * launch whose pieces merge in-kernel; larger ones as a prepare, a stream-K and a merge
 * launch.
 * Key p of sequence b contributes iff p < seq_len[b] and p <= query_pos[b]
 * (gqa_attention_wrapper.v:279); rows outside that range are never read.
 * Lengths are read on the device: an entry violating the rules of
 * gqa_validate_lengths yields NaN rows for that sequence (never an out-of-range read).
 * Replaces CTRL.start of axi_lite_regs.v:147-151 and the stream/egress contract. */
int gqa_decode_bf16(const gqa_params_t* params, const uint16_t* q, const uint16_t* k,
                    const uint16_t* v, const gqa_kv_layout_t* kv, const int32_t* seq_len,
                    const int32_t* query_pos, int32_t batch, uint16_t* out, void* workspace,
                    size_t workspace_bytes, void* stream);

/* gqa_decode_bf16 without a workspace argument, allocating nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same arguments (less the
 * workspace), results and rules as gqa_decode_bf16.  The workspace is a 32 MiB device array
 * inside the library, one copy per GPU, held until the process ends; the first call on a
 * GPU looks up its address and clears its counters with a fill kernel on `stream`.  A batch
 * whose decode workspace does not fit (about 440 sequences of any capacity on a 256-CU
 * GPU; gqa_decode_workspace_bytes gives the size) is rejected with GQA_ERR_WORKSPACE before
 * any launch.  Every call on a GPU shares that array and leaves it as its plan did: calls
 * that overlap on one GPU (other streams or threads) race, so callers order them. */
int gqa_decode_bf16_noalloc(const gqa_params_t* params, const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, const gqa_kv_layout_t* kv, const int32_t* seq_len,
                            const int32_t* query_pos, int32_t batch, uint16_t* out, void* stream);

/* Paged cache: a pool of blocks of 16 positions (the core's KV_BLOCK_LEN,
 * gqa_controller.v:20); block j of sequence b is pool block block_table[b*max_blocks + j],
 * and row (block id, KV head h, position-in-block r) starts at element
 * id*block_stride + h*head_stride + r*pos_stride (each row 128 contiguous BF16, strides
 * multiples of 8, pools 16-byte aligned).  [n_blocks][8][16][128] is the natural pool. */
typedef struct gqa_paged_kv {
    int64_t block_stride;
    int64_t head_stride;
    int64_t pos_stride;
    int32_t block_size;   /* must be 16 */
    int32_t max_blocks;   /* block-table entries per sequence; capacity = 16 * max_blocks */
    int32_t n_blocks;     /* blocks in the pool */
} gqa_paged_kv_t;

/* Workspace bytes gqa_decode_paged_bf16 needs.  0 if the configuration is invalid. */
size_t gqa_decode_paged_workspace_bytes(const gqa_params_t* params, int32_t batch, int32_t max_blocks);

/* gqa_decode_bf16 over a paged cache: same arguments, results and rules, with the K/V
 * pools and the block table (device, int32 [batch][max_blocks]) in place of the
 * contiguous cache.  A block id outside [0, n_blocks) for a row the sequence needs gives
 * NaN rows for that sequence (never an out-of-range read).  The workspace needs no
 * particular contents.  Replaces the same start of axi_lite_regs.v:147-151, with the
 * K/V stream fed block by block as the core's KV_BLOCK_LEN tiles. */
int gqa_decode_paged_bf16(const gqa_params_t* params, const uint16_t* q, const uint16_t* k_pool,
                          const uint16_t* v_pool, const gqa_paged_kv_t* kv, const int32_t* block_table,
                          const int32_t* seq_len, const int32_t* query_pos, int32_t batch, uint16_t* out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* gqa_kv_append_bf16 into a paged cache: rows go to block block_table[b][(start+t)/16],
 * row (start+t)%16; rows whose block id is outside [0, n_blocks) are not written. */
int gqa_kv_append_paged_bf16(const gqa_params_t* params, const uint16_t* k_new, const uint16_t* v_new,
                             uint16_t* k_pool, uint16_t* v_pool, const gqa_paged_kv_t* kv,
                             const int32_t* block_table, const int32_t* start, int32_t batch, int32_t n_new,
                             void* stream);

/* Chunked prefill: n_new query tokens per sequence, appended after start[b] cached
 * positions (the reference core computes one token per start; a chunk is that step for
 * tokens at positions start[b] .. start[b]+n_new-1 of one sequence,
 * gen_gqa_wrapper_vectors.py:121-139 per token):
 *   q          [batch][n_new][32][128]  Q rows of the chunk's tokens (unrotated; rotated at
 *              their positions when GQA_ROPE_Q)
 *   k_new, v_new [batch][n_new][8][128]  the chunk's K and V rows (K rotated at its
 *              position when GQA_ROPE_K)
 *   k_cache, v_cache  cache per `kv`; rows at positions < start[b] are read as stored
 *              (post-RoPE); the call writes the chunk's rows at start[b] + t (K rotated
 *              and rounded double -> f32 -> BF16, V as given) before it attends
 *   start      [batch] int32, device; 0 <= start[b] <= capacity - n_new, else that
 *              sequence's output rows are NaN and its cache is not written
 *   out        [batch][n_new][32][128]
 *   workspace  gqa_prefill_workspace_bytes(params, batch, n_new, kv->capacity) bytes (any
 *              contents)
 * Token t attends to keys p <= start[b] + t (gqa_attention_wrapper.v:279 per token), the
 * chunk's own keys carried to ~24 bits (their rotated value is not re-rounded, as in the
 * golden).  Replaces the reference's per-token start loop for a run of tokens.
 * Chunks of at most 16 new tokens (multi-token decode: drafts, a few steps at once) split
 * the keys of every (sequence, KV head) over all CUs and merge per-range partials (three
 * launches: preparation, which also appends the chunk's rows, stream, merge); longer chunks
 * run the KV append, a staging kernel that copies the K/V rows the attention reads into
 * fp16 planes in the workspace (a power-of-two scale per 64-position block, so BF16 values
 * convert exactly), and one attention kernel over 32-token query blocks.  Every path ends
 * with an fp64 recomputation of the output rows its kernels may have computed outside 64
 * BF16 ULP.  GQA_PLAN_NO_MULTI_TOKEN sends short chunks to the attention kernel too.  For
 * longer chunks the workspace grows with capacity (the staging planes hold 512 bytes per
 * position of every (sequence, KV head): 143 MB for batch 4 over 8704 positions). */
size_t gqa_prefill_workspace_bytes(const gqa_params_t* params, int32_t batch, int32_t n_new,
                                   int32_t capacity);

int gqa_prefill_bf16(const gqa_params_t* params, const uint16_t* q, const uint16_t* k_new,
                     const uint16_t* v_new, uint16_t* k_cache, uint16_t* v_cache,
                     const gqa_kv_layout_t* kv, const int32_t* start, int32_t batch, int32_t n_new,
                     uint16_t* out, void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference (measurement): byte offset, within a prefill workspace of
 * gqa_prefill_workspace_bytes(params, batch, n_new, capacity) bytes, of the uint32 count of
 * output rows the last gqa_prefill_bf16 call on it recomputed in fp64 (read it after the
 * call's stream has finished).  0 for arguments gqa_prefill_workspace_bytes rejects. */
size_t gqa_prefill_rescored_rows_offset(const gqa_params_t* params, int32_t batch, int32_t n_new,
                                        int32_t capacity);

/* KV append with RoPE on insert: writes k_new / v_new ([batch][n_new][8][128]) into the
 * cache at positions start[b] + t, K rotated at its position when GQA_ROPE_K and rounded
 * double -> f32 -> BF16 (the rope_unit's role in gqa_attention_wrapper.v:302-308 for a
 * cache kept post-RoPE; rounding pyfiles/gqa_reference.py:15-19).  Sequences with
 * start[b] outside [0, capacity - n_new] are skipped.  The step before a decode call on a
 * post-RoPE cache. */
int gqa_kv_append_bf16(const gqa_params_t* params, const uint16_t* k_new, const uint16_t* v_new,
                       uint16_t* k_cache, uint16_t* v_cache, const gqa_kv_layout_t* kv,
                       const int32_t* start, int32_t batch, int32_t n_new, void* stream);

/* rope_unit in isolation (rope_unit.v:38-330 as tests/tb_rope_unit.sv drives it;
 * golden pyfiles/gen_rope_test_vectors.py:16-20): out[r] = BF16(rope(in[r], position)),
 * position = positions[r] if positions != NULL (device int32) else pos0 + r.
 * Rows are 128 BF16 with row stride `row_stride` elements (in and out). */
int gqa_rope_rows_bf16(const uint16_t* in, uint16_t* out, int64_t n_rows, int64_t row_stride,
                       const int32_t* positions, int32_t pos0, double theta, void* stream);

/* Kernel timing for measurement harnesses.  While enabled, each decode or prefill
 * call brackets its kernels with HIP events on the call's stream (up to `max_calls`
 * calls are recorded; later ones are not), in up to four stages: decode {stream kernel,
 * merge kernel} (the Q-operand preparation kernel runs before the first event), prefill
 * {KV append, staging and reduce kernels; attention kernel; fp64 rescore}, prefill of at
 * most 16 new tokens {preparation kernel (with the append); stream kernel; merge kernel;
 * fp64 rescore}.  gqa_profile_read waits for the recorded events, returns the summed times
 * of the first two stages and the number of calls recorded, and clears the record;
 * gqa_profile_read_stages does the same for up to four stages (a path's missing stages
 * read 0).  Not for the hot path: enabling creates the events.  No reference counterpart
 * (the reference's timing is its simulator's cycle count). */
typedef struct gqa_profile {
    double kernel_ms[2];  /* summed durations of the call's first and second kernel */
    int32_t calls;        /* calls recorded */
} gqa_profile_t;

int gqa_profile_enable(int32_t max_calls); /* max_calls <= 0 disables and frees */
int gqa_profile_read(gqa_profile_t* out);
/* stage_ms[i], i < n_stages <= 4: summed time of stage i over the recorded calls (ABI 4.1). */
int gqa_profile_read_stages(double* stage_ms, int32_t n_stages, int32_t* calls);

/* Human-readable name of a status code. */
const char* gqa_status_string(int status);

/* ABI version: (major << 16) | minor. */
uint32_t gqa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GQA_H */

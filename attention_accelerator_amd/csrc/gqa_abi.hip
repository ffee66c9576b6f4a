// gqa_abi.hip -- the extern "C" surface of libgqa.so (declared in include/gqa.h).
//
// Validation mirrors the reference core's start-time rejection
// (gqa_attention_wrapper.v:230-244): a rejected call launches nothing and writes no
// output, and the status says why.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "gqa.h"
#include "gqa_internal.h"

namespace gqa {

void fill_rope_table(double theta, RopeTable* t) {
    // angle = position * theta ** (-2.0 * i / 128), pyfiles/gen_gqa_wrapper_vectors.py:30.
    for (int i = 0; i < kPairs; ++i) t->inv_freq[i] = std::pow(theta, (-2.0 * i) / kD);
}

namespace {

// Persistent workgroups of the decode stream kernel: one wave each, one per SIMD (four
// per CU) of the current device -- 1024 on the 256 CUs of an MI355X.  Measured on
// MI355X, one wave per SIMD streams faster than two (fewer concurrent DRAM streams; the
// kernel's ~250 registers leave room for one wave per SIMD anyway).  1024 when no
// device answers.  gqa_params_t.stream_wgs overrides it (tuning and tests).
constexpr int32_t kStreamWgsDefault = 1024;
constexpr int32_t kWavesPerCu = 4;

// Batches whose caches hold at most this many keys in all (B * 8 * capacity; 128 MB of
// K/V) run as one launch (decode_single_kernel): for them the three dependent launches of
// the stream path cost more than the HBM traffic.  GQA_PLAN_STREAM_K turns it off.
constexpr int64_t kSingleLaunchMaxKeys = int64_t{1} << 18;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int32_t device_stream_wgs() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
        (void)hipGetLastError();   // leave no error behind for the caller's next HIP call
        return kStreamWgsDefault;
    }
    return cus * kWavesPerCu;
}

int32_t stream_wgs(const gqa_params_t* p) { return p->stream_wgs > 0 ? p->stream_wgs : device_stream_wgs(); }

// Chunks of at most kMultiMaxNew new tokens take the multi-token path (stream-K over the
// keys, prefill arithmetic); GQA_PLAN_NO_MULTI_TOKEN sends them through the prefill
// attention kernel instead.
bool use_multi(const gqa_params_t* p, int32_t n_new) {
    return n_new <= kMultiMaxNew && (p->flags & GQA_PLAN_NO_MULTI_TOKEN) == 0u;
}

// XCD weighting of the stream-K ranges, per mille of a range moved from each workgroup on
// an odd XCD to its even neighbour; GQA_XCD_SKEW overrides the path's default (0 gives
// equal ranges).  At most 250: an odd range keeps at least 3/4 of the range size, more
// than a segment lead.  Measured defaults (B=64 ragged 512-8192): 80 for the one-wave
// multi-token kernel (T <= 4: 0 / 40 / 80 / 120 / 160 gave 226.0 / 223.6 / 221.8 / 225.0 /
// 228.1 us per step, two boxes), 40 for the two-wave one (T <= 8, two waves per SIMD: 259.9 /
// 256.1 / 260.8 us at 0 / 40 / 80), 0 for the four-wave one (T <= 16: 40 made it 375 -> 379
// us) and for decode (30 made it 187.6 -> 191 us).
int32_t xcd_skew_pm(int32_t dflt) {
    const char* s = std::getenv("GQA_XCD_SKEW");
    if (s) {
        const int v = std::atoi(s);
        if (v >= 0 && v <= 250) return v;
    }
    return dflt;
}

// Workgroups of the multi-token stream kernel: multi_simd_waves(n_new) waves per SIMD,
// multi_waves(n_new) waves per workgroup.
int32_t multi_wgs(const gqa_params_t* p, int32_t n_new) {
    const int32_t w = stream_wgs(p) * multi_simd_waves(n_new) / multi_waves(n_new);
    return w > 0 ? w : 1;
}

bool geometry_ok(const gqa_params_t* p) {
    if (p->n_q_heads != kHq || p->n_kv_heads != kHkv || p->head_dim != kD) return false;
    if (!(p->scale != 0.0) || !std::isfinite(p->scale)) return false;
    if ((p->flags & ~(GQA_ROPE_Q | GQA_ROPE_K | GQA_PLAN_STREAM_K | GQA_PLAN_NO_MULTI_TOKEN)) != 0) return false;
    if (p->stream_wgs < 0 || p->stream_wgs > kStreamWgsMax) return false;
    if ((p->flags & (GQA_ROPE_Q | GQA_ROPE_K)) && !(p->rope_theta > 0.0 && std::isfinite(p->rope_theta)))
        return false;
    return true;
}

// The score scale folded into Q: scale * log2(e) in double, so that exp(scale * q.k - max)
// becomes exp2 of the folded score.
double qk_scale_log2(const gqa_params_t* p) { return p->scale * 1.4426950408889634; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Opt-in kernel timing (gqa_profile_enable / gqa_profile_read / gqa_profile_read_stages).
struct Profiler {
    std::mutex mu;
    std::vector<hipEvent_t> events;   // kProfileEvents per recorded call
    int32_t capacity = 0;
    int32_t used = 0;
};

Profiler& profiler() {
    static Profiler p;
    return p;
}

// Returns the next free set of kProfileEvents events, or nullptr when profiling is off or full.
hipEvent_t* profile_slot() {
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    if (p.used >= p.capacity) return nullptr;
    return &p.events[static_cast<size_t>(p.used++) * kProfileEvents];
}

}  // namespace

DecodePlan plan_decode(const gqa_params_t* params, int32_t batch, int32_t capacity, bool paged,
                       int64_t max_single_segments) {
    DecodePlan plan{};
    plan.n_wgs = stream_wgs(params);
    const int64_t keys_cap = static_cast<int64_t>(batch) * kHkv * capacity;
    const bool single_fits = max_single_segments < 0 || static_cast<int64_t>(batch) * kHkv <= max_single_segments;
    if (!paged && (params->flags & GQA_PLAN_STREAM_K) == 0u && keys_cap <= kSingleLaunchMaxKeys && single_fits) {
        // Single launch: about one 4-wave workgroup per CU (n_wgs / 4), pieces of at least
        // 256 keys (64 per wave: below that the last piece's merge of more partials costs
        // more than the shorter streams save; B=1 L=4096 runs in 18.7 us with 256-key pieces,
        // 20.7 us with 128) in multiples of 64, sized from the capacity (the lengths live on
        // the device); pieces past a sequence's length exit at once.
        const int64_t n_pieces = plan.n_wgs / 4 > 0 ? plan.n_wgs / 4 : 1;
        int64_t pk = (keys_cap + n_pieces - 1) / n_pieces;
        pk = pk < 256 ? 256 : (pk + 63) / 64 * 64;
        plan.piece_keys = static_cast<int32_t>(pk);
        plan.pieces_cap = static_cast<int32_t>((capacity + pk - 1) / pk);
        plan.n_slots = static_cast<int64_t>(batch) * kHkv * plan.pieces_cap;
    } else {
        plan.n_slots = static_cast<int64_t>(plan.n_wgs) + static_cast<int64_t>(kHkv) * batch;
        plan.q_op_bytes = static_cast<size_t>(batch) * kHkv * kGroup * kD * sizeof(double);
        plan.plan_bytes = 256 + align_up((static_cast<size_t>(batch) + 1) * sizeof(int64_t), 256) +
                          align_up(static_cast<size_t>(batch) * sizeof(int32_t), 256);
    }
    plan.part_o_bytes = align_up(static_cast<size_t>(plan.n_slots) * kGroup * kD * sizeof(double), 256);
    plan.part_ml_bytes = align_up(static_cast<size_t>(plan.n_slots) * kGroup * sizeof(double2), 256);
    plan.count_bytes = align_up(static_cast<size_t>(batch) * kHkv * sizeof(unsigned long long), 256);
    plan.workspace_bytes =
        plan.part_o_bytes + plan.part_ml_bytes + plan.q_op_bytes + plan.plan_bytes + plan.count_bytes;
    return plan;
}

// Rescore region of a prefill or multi-token workspace: header, flagged rows, per-row piece
// counters, the chunk's cos/sin table, partial slots, the per-row running maxima and the key
// and V statistics the flag decision reads (ncb chunk blocks of nr rows of prefix maxima).
namespace {
struct RsLayout {
    size_t flat, rows, gcnt, done, cs, part_o, part_ml, m, kc, dc, kpre, dpre, kblk, dblk, total;
};

RsLayout rs_layout(int32_t batch, int32_t n_new, int32_t ncb, int32_t nr, int32_t nblk) {
    const size_t rows = static_cast<size_t>(batch) * n_new * kHq;
    const size_t toks = static_cast<size_t>(batch) * n_new;
    const size_t bh = static_cast<size_t>(batch) * kHkv;
    const size_t pre = bh * static_cast<size_t>(ncb) * static_cast<size_t>(nr);
    RsLayout l{};
    l.flat = 256;
    l.rows = l.flat + align_up(rows * sizeof(uint32_t), 256);
    l.gcnt = l.rows + align_up(rows * sizeof(uint32_t), 256);
    l.done = l.gcnt + align_up(bh * sizeof(uint32_t), 256);
    l.cs = l.done + align_up(rows * sizeof(uint32_t), 256);
    l.part_o = l.cs + align_up(toks * kPairs * sizeof(double2), 256);
    l.part_ml = l.part_o + align_up(size_t{kRsSlots} * kGroup * kD * sizeof(double), 256);
    l.m = l.part_ml + align_up(size_t{kRsSlots} * kGroup * sizeof(double2), 256);
    l.kc = l.m + align_up(rows * sizeof(float), 256);
    l.dc = l.kc + align_up(bh * static_cast<size_t>(ncb) * 8 * sizeof(uint32_t), 256);
    l.kpre = l.dc + align_up(bh * static_cast<size_t>(ncb) * kD * sizeof(uint32_t), 256);
    l.dpre = l.kpre + align_up(pre * 8 * sizeof(uint32_t), 256);
    l.kblk = l.dpre + align_up(pre * kD * sizeof(uint16_t), 256);
    l.dblk = l.kblk + align_up(bh * static_cast<size_t>(nblk) * 8 * sizeof(uint32_t), 256);
    l.total = l.dblk + align_up(bh * static_cast<size_t>(nblk) * (kD / 2) * sizeof(uint32_t), 256);
    return l;
}
}  // namespace

size_t rescore_bytes(int32_t batch, int32_t n_new, int32_t ncb, int32_t nr, int32_t nblk) {
    return rs_layout(batch, n_new, ncb, nr, nblk).total;
}

void rescore_layout(PrefillArgs& a, const gqa_params_t* params, void* base, int32_t ncb, int32_t nr, int32_t nblk) {
    const RsLayout l = rs_layout(a.batch, a.n_new, ncb, nr, nblk);
    char* p = static_cast<char*>(base);
    a.rs_hdr = reinterpret_cast<uint32_t*>(p);
    a.rs_flat = reinterpret_cast<uint32_t*>(p + l.flat);
    a.rs_rows = reinterpret_cast<uint32_t*>(p + l.rows);
    a.rs_gcnt = reinterpret_cast<uint32_t*>(p + l.gcnt);
    a.rs_done = reinterpret_cast<uint32_t*>(p + l.done);
    a.rs_cs = reinterpret_cast<double2*>(p + l.cs);
    a.rs_part_o = reinterpret_cast<double*>(p + l.part_o);
    a.rs_part_ml = reinterpret_cast<double2*>(p + l.part_ml);
    a.rs_m = reinterpret_cast<float*>(p + l.m);
    a.rs_kc = reinterpret_cast<uint32_t*>(p + l.kc);
    a.rs_dc = reinterpret_cast<uint32_t*>(p + l.dc);
    a.rs_kpre = reinterpret_cast<uint32_t*>(p + l.kpre);
    a.rs_dpre = reinterpret_cast<uint16_t*>(p + l.dpre);
    a.rs_ncb = ncb;
    a.rs_nr = nr;
    a.rs_kblk = reinterpret_cast<uint32_t*>(p + l.kblk);
    a.rs_dblk = reinterpret_cast<uint32_t*>(p + l.dblk);
    a.rs_nblk = nblk;
    // One-wave workgroups, one per SIMD (the kernel's registers allow one wave per SIMD):
    // the flagged rows' tiles are cut into about as many (tile, piece) pairs as run at once.
    const int32_t wgs = stream_wgs(params);
    a.rs_wgs = wgs < 1 ? 1 : wgs > static_cast<int32_t>(kRsSlots) ? static_cast<int32_t>(kRsSlots) : wgs;
}

}  // namespace gqa

using namespace gqa;

extern "C" {

uint32_t gqa_abi_version(void) { return (4u << 16) | 1u; }

const char* gqa_status_string(int status) {
    switch (status) {
        case GQA_OK: return "ok";
        case GQA_ERR_INVALID_CONFIG: return "invalid configuration";
        case GQA_ERR_BAD_POINTER: return "null or misaligned pointer or stride";
        case GQA_ERR_WORKSPACE: return "workspace missing or too small";
        case GQA_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

int gqa_validate_registers(int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           int32_t tile_dim, int32_t seq_len, int32_t n_kv_tiles,
                           int32_t kv_block_len, uint16_t scale_bf16) {
    if (n_q_heads != kHq || n_kv_heads != kHkv || head_dim != kD || tile_dim != 16)
        return GQA_ERR_INVALID_CONFIG;
    if (kv_block_len <= 0 || seq_len <= 0) return GQA_ERR_INVALID_CONFIG;
    const int64_t want_tiles = (static_cast<int64_t>(seq_len) + kv_block_len - 1) / kv_block_len;
    if (n_kv_tiles != want_tiles) return GQA_ERR_INVALID_CONFIG;
    if (scale_bf16 == 0) return GQA_ERR_INVALID_CONFIG;
    return GQA_OK;
}

int gqa_validate_lengths(const int32_t* seq_len, const int32_t* query_pos, int32_t batch,
                         int32_t capacity) {
    if (!seq_len || !query_pos) return GQA_ERR_BAD_POINTER;
    if (batch <= 0 || capacity <= 0) return GQA_ERR_INVALID_CONFIG;
    for (int32_t b = 0; b < batch; ++b) {
        if (seq_len[b] < 1 || seq_len[b] > capacity) return GQA_ERR_INVALID_CONFIG;
        if (query_pos[b] < 0 || query_pos[b] >= seq_len[b]) return GQA_ERR_INVALID_CONFIG;
    }
    return GQA_OK;
}

size_t gqa_decode_workspace_bytes(const gqa_params_t* params, int32_t batch, int32_t capacity) {
    if (!params || !geometry_ok(params) || batch <= 0 || capacity <= 0) return 0;
    return plan_decode(params, batch, capacity).workspace_bytes;
}

}  // extern "C"

namespace {

// Common tail of the contiguous and paged decode entry points: workspace carve-up and launch.
// `counters`: the per-segment piece counters of the one-launch paths, when they live outside
// the workspace (nullptr: at the end of the workspace, as gqa_decode_workspace_bytes counts).
int decode_launch(const DecodePlan& plan, const gqa_params_t* params, const uint16_t* q, const uint16_t* k,
                  const uint16_t* v, int64_t s0, int64_t s1, int64_t s2, int32_t capacity,
                  const int32_t* block_table, int32_t max_blocks, int32_t n_blocks, const int32_t* seq_len,
                  const int32_t* query_pos, int32_t batch, uint16_t* out, void* workspace,
                  size_t workspace_bytes, void* stream, unsigned long long* counters = nullptr) {
    const size_t need = counters ? plan.workspace_bytes - plan.count_bytes : plan.workspace_bytes;
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256)) return GQA_ERR_WORKSPACE;

    DecodeArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.seq_len = seq_len;
    a.query_pos = query_pos;
    a.out = out;
    char* ws = static_cast<char*>(workspace);
    a.part_o = reinterpret_cast<double*>(ws);
    a.part_ml = reinterpret_cast<double2*>(ws + plan.part_o_bytes);
    a.q_op = reinterpret_cast<double*>(ws + plan.part_o_bytes + plan.part_ml_bytes);
    char* pl = ws + plan.part_o_bytes + plan.part_ml_bytes + plan.q_op_bytes;
    a.plan_hdr = reinterpret_cast<int64_t*>(pl);
    a.seq_off = reinterpret_cast<int64_t*>(pl + 256);
    a.seq_nreal = reinterpret_cast<int32_t*>(pl + 256 + align_up((static_cast<size_t>(batch) + 1) * sizeof(int64_t), 256));
    a.seg_count = counters ? counters : reinterpret_cast<unsigned long long*>(pl + plan.plan_bytes);
    a.pieces_cap = plan.pieces_cap;
    a.piece_keys = plan.piece_keys;
    a.block_table = block_table;
    a.max_blocks = max_blocks;
    a.n_blocks = n_blocks;
    a.kv_batch_stride = s0;
    a.kv_head_stride = s1;
    a.kv_pos_stride = s2;
    a.capacity = capacity;
    a.batch = batch;
    a.n_wgs = plan.n_wgs;
    a.skew_pm = xcd_skew_pm(0);
    a.qk_scale_log2 = qk_scale_log2(params);
    a.flags = params->flags;
    fill_rope_table(params->rope_theta, &a.rope);
    const hipError_t e = launch_decode(a, batch, static_cast<hipStream_t>(stream), profile_slot());
    return e == hipSuccess ? GQA_OK : GQA_ERR_HIP;
}

bool paged_layout_ok(const gqa_paged_kv_t* kv) {
    return kv->block_size == 16 && kv->max_blocks > 0 && kv->n_blocks > 0 && kv->pos_stride >= kD &&
           kv->head_stride >= 0 && kv->block_stride >= 0 &&
           static_cast<int64_t>(kv->max_blocks) * 16 <= 0x7FFFFFFF;
}

// Argument checks of the contiguous-cache decode entry points (nothing is launched on error).
int decode_args_status(const gqa_params_t* params, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const gqa_kv_layout_t* kv, const int32_t* seq_len, const int32_t* query_pos,
                       int32_t batch, const uint16_t* out) {
    if (!params || !kv) return GQA_ERR_BAD_POINTER;
    if (!geometry_ok(params)) return GQA_ERR_INVALID_CONFIG;
    if (batch <= 0 || kv->capacity <= 0) return GQA_ERR_INVALID_CONFIG;
    if (kv->pos_stride < kD || kv->head_stride < 0 || kv->batch_stride < 0)
        return GQA_ERR_INVALID_CONFIG;
    if (!q || !k || !v || !out || !seq_len || !query_pos) return GQA_ERR_BAD_POINTER;
    if (!aligned(q, 2) || !aligned(out, 4) || !aligned(k, 16) || !aligned(v, 16) ||
        !aligned(seq_len, 4) || !aligned(query_pos, 4))
        return GQA_ERR_BAD_POINTER;
    if (kv->pos_stride % 8 || kv->head_stride % 8 || kv->batch_stride % 8) return GQA_ERR_BAD_POINTER;
    // Rows of one (sequence, KV head) are addressed with 32-bit byte offsets, which run
    // up to 64 rows past the last valid one (prefetch offsets, clamped before use).
    if ((static_cast<uint64_t>(kv->capacity) + 64u) * static_cast<uint64_t>(kv->pos_stride) * 2u >
        0xFFFFFF00ull)
        return GQA_ERR_INVALID_CONFIG;
    return GQA_OK;
}

// ---- The decode entry point that allocates nothing (gqa_decode_bf16_noalloc): its
// workspace is this file-scope device array, one copy per GPU, held until the process ends.
// The first kNoAllocCountBytes hold the per-segment counters of the one-launch paths
// (they must read zero between calls; every call leaves them so), the rest the plan's
// partials, Q operands and plan.  Calls on one GPU share it: calls that overlap race.
constexpr size_t kNoAllocScratchBytes = size_t{32} << 20;
constexpr size_t kNoAllocCountBytes = size_t{64} << 10;            // 8192 segments
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};    // device address of `scratch` on each GPU (set-up done)

// Device address of the current GPU's scratch.  The first call on a GPU looks the address
// up (hipGetSymbolAddress, with that GPU current) and clears the counter region with a fill
// kernel on `stream` (no memset, so the call may sit in a captured graph).  nullptr and a
// status on failure.
void* noalloc_scratch(hipStream_t stream, int& status) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        status = GQA_ERR_HIP;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            status = GQA_ERR_HIP;
            return nullptr;
        }
        if (launch_zero_words(static_cast<uint32_t*>(ptr), static_cast<int64_t>(kNoAllocCountBytes / 4), stream) !=
            hipSuccess) {
            status = GQA_ERR_HIP;
            return nullptr;
        }
        g_scratch_dev[dev] = ptr;
    }
    status = GQA_OK;
    return g_scratch_dev[dev];
}

}  // namespace

extern "C" {

int gqa_decode_bf16(const gqa_params_t* params, const uint16_t* q, const uint16_t* k,
                    const uint16_t* v, const gqa_kv_layout_t* kv, const int32_t* seq_len,
                    const int32_t* query_pos, int32_t batch, uint16_t* out, void* workspace,
                    size_t workspace_bytes, void* stream) {
    const int st = decode_args_status(params, q, k, v, kv, seq_len, query_pos, batch, out);
    if (st != GQA_OK) return st;
    return decode_launch(plan_decode(params, batch, kv->capacity), params, q, k, v, kv->batch_stride, kv->head_stride,
                         kv->pos_stride, kv->capacity,
                         nullptr, 0, 0, seq_len, query_pos, batch, out, workspace, workspace_bytes, stream);
}

int gqa_decode_bf16_noalloc(const gqa_params_t* params, const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, const gqa_kv_layout_t* kv, const int32_t* seq_len,
                            const int32_t* query_pos, int32_t batch, uint16_t* out, void* stream) {
    int st = decode_args_status(params, q, k, v, kv, seq_len, query_pos, batch, out);
    if (st != GQA_OK) return st;
    const DecodePlan plan =
        plan_decode(params, batch, kv->capacity, false, static_cast<int64_t>(kNoAllocCountBytes / sizeof(unsigned long long)));
    if (plan.workspace_bytes - plan.count_bytes > kNoAllocScratchBytes - kNoAllocCountBytes) return GQA_ERR_WORKSPACE;
    char* base = static_cast<char*>(noalloc_scratch(static_cast<hipStream_t>(stream), st));
    if (!base) return st;
    return decode_launch(plan, params, q, k, v, kv->batch_stride, kv->head_stride, kv->pos_stride, kv->capacity,
                         nullptr, 0, 0, seq_len, query_pos, batch, out, base + kNoAllocCountBytes,
                         kNoAllocScratchBytes - kNoAllocCountBytes, stream,
                         reinterpret_cast<unsigned long long*>(base));
}

size_t gqa_decode_paged_workspace_bytes(const gqa_params_t* params, int32_t batch, int32_t max_blocks) {
    if (!params || !geometry_ok(params) || batch <= 0 || max_blocks <= 0 ||
        static_cast<int64_t>(max_blocks) * 16 > 0x7FFFFFFF)
        return 0;
    return plan_decode(params, batch, max_blocks * 16, true).workspace_bytes;
}

int gqa_decode_paged_bf16(const gqa_params_t* params, const uint16_t* q, const uint16_t* k_pool,
                          const uint16_t* v_pool, const gqa_paged_kv_t* kv, const int32_t* block_table,
                          const int32_t* seq_len, const int32_t* query_pos, int32_t batch, uint16_t* out,
                          void* workspace, size_t workspace_bytes, void* stream) {
    if (!params || !kv) return GQA_ERR_BAD_POINTER;
    if (!geometry_ok(params) || batch <= 0 || !paged_layout_ok(kv)) return GQA_ERR_INVALID_CONFIG;
    if (!q || !k_pool || !v_pool || !out || !seq_len || !query_pos || !block_table) return GQA_ERR_BAD_POINTER;
    if (!aligned(q, 2) || !aligned(out, 4) || !aligned(k_pool, 16) || !aligned(v_pool, 16) ||
        !aligned(seq_len, 4) || !aligned(query_pos, 4) || !aligned(block_table, 4))
        return GQA_ERR_BAD_POINTER;
    if (kv->pos_stride % 8 || kv->head_stride % 8 || kv->block_stride % 8) return GQA_ERR_BAD_POINTER;
    return decode_launch(plan_decode(params, batch, kv->max_blocks * 16, true), params, q, k_pool, v_pool,
                         kv->block_stride, kv->head_stride, kv->pos_stride,
                         kv->max_blocks * 16, block_table, kv->max_blocks, kv->n_blocks, seq_len, query_pos,
                         batch, out, workspace, workspace_bytes, stream);
}

int gqa_profile_enable(int32_t max_calls) {
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    for (hipEvent_t e : p.events)
        if (e) (void)hipEventDestroy(e);
    p.events.clear();
    p.capacity = 0;
    p.used = 0;
    if (max_calls <= 0) return GQA_OK;
    p.events.resize(static_cast<size_t>(max_calls) * kProfileEvents);
    for (auto& e : p.events) {
        if (hipEventCreate(&e) != hipSuccess) {
            e = nullptr;
            return GQA_ERR_HIP;
        }
    }
    p.capacity = max_calls;
    return GQA_OK;
}

int gqa_profile_read_stages(double* stage_ms, int32_t n_stages, int32_t* calls) {
    if (!stage_ms || n_stages < 0 || n_stages > kProfileEvents - 1) return GQA_ERR_BAD_POINTER;
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    double sum[kProfileEvents - 1] = {};
    for (int32_t i = 0; i < p.used; ++i) {
        hipEvent_t* ev = &p.events[static_cast<size_t>(i) * kProfileEvents];
        if (hipEventSynchronize(ev[kProfileEvents - 1]) != hipSuccess) return GQA_ERR_HIP;
        for (int j = 0; j + 1 < kProfileEvents; ++j) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, ev[j], ev[j + 1]) != hipSuccess) return GQA_ERR_HIP;
            sum[j] += ms;
        }
    }
    for (int j = 0; j < n_stages; ++j) stage_ms[j] = sum[j];
    if (calls) *calls = p.used;
    p.used = 0;
    return GQA_OK;
}

int gqa_profile_read(gqa_profile_t* out) {
    if (!out) return GQA_ERR_BAD_POINTER;
    double st[2] = {0.0, 0.0};
    int32_t n = 0;
    const int rc = gqa_profile_read_stages(st, 2, &n);
    if (rc != GQA_OK) return rc;
    out->kernel_ms[0] = st[0];
    out->kernel_ms[1] = st[1];
    out->calls = n;
    return GQA_OK;
}

int gqa_decode_workspace_init(const gqa_params_t* params, int32_t batch, int32_t capacity,
                              void* workspace, size_t workspace_bytes, void* stream) {
    if (!params) return GQA_ERR_BAD_POINTER;
    if (!geometry_ok(params) || batch <= 0 || capacity <= 0) return GQA_ERR_INVALID_CONFIG;
    const DecodePlan plan = plan_decode(params, batch, capacity);
    if (!workspace || workspace_bytes < plan.workspace_bytes || !aligned(workspace, 256))
        return GQA_ERR_WORKSPACE;
    const hipError_t e = launch_zero_words(static_cast<uint32_t*>(workspace),
                                           static_cast<int64_t>(plan.workspace_bytes / 4),
                                           static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GQA_OK : GQA_ERR_HIP;
}

int gqa_rope_rows_bf16(const uint16_t* in, uint16_t* out, int64_t n_rows, int64_t row_stride,
                       const int32_t* positions, int32_t pos0, double theta, void* stream) {
    if (n_rows < 0 || row_stride < kD || !(theta > 0.0 && std::isfinite(theta)))
        return GQA_ERR_INVALID_CONFIG;
    if (n_rows == 0) return GQA_OK;
    if (!in || !out) return GQA_ERR_BAD_POINTER;
    if (!aligned(in, 2) || !aligned(out, 2) || (positions && !aligned(positions, 4)))
        return GQA_ERR_BAD_POINTER;
    if (n_rows > (int64_t{1} << 31)) return GQA_ERR_INVALID_CONFIG;
    RopeArgs a{};
    a.in = in;
    a.out = out;
    a.positions = positions;
    a.n_rows = n_rows;
    a.row_stride = row_stride;
    a.pos0 = pos0;
    fill_rope_table(theta, &a.rope);
    const hipError_t e = launch_rope_rows(a, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GQA_OK : GQA_ERR_HIP;
}

}  // extern "C"

namespace {

// Checks shared by the prefill and append entry points; fills the argument block.
int prefill_args(const gqa_params_t* params, const uint16_t* k_new, const uint16_t* v_new,
                 uint16_t* k_cache, uint16_t* v_cache, const gqa_kv_layout_t* kv, const int32_t* start,
                 int32_t batch, int32_t n_new, PrefillArgs& a) {
    if (!params || !kv) return GQA_ERR_BAD_POINTER;
    if (!geometry_ok(params)) return GQA_ERR_INVALID_CONFIG;
    if (batch <= 0 || n_new <= 0 || kv->capacity < n_new) return GQA_ERR_INVALID_CONFIG;
    if (kv->pos_stride < kD || kv->head_stride < 0 || kv->batch_stride < 0) return GQA_ERR_INVALID_CONFIG;
    if (!k_new || !v_new || !k_cache || !v_cache || !start) return GQA_ERR_BAD_POINTER;
    if (!aligned(k_new, 2) || !aligned(v_new, 2) || !aligned(k_cache, 16) || !aligned(v_cache, 16) ||
        !aligned(start, 4))
        return GQA_ERR_BAD_POINTER;
    if (kv->pos_stride % 8 || kv->head_stride % 8 || kv->batch_stride % 8) return GQA_ERR_BAD_POINTER;
    // The attention kernel addresses the rows of a 64-key block with 32-bit byte offsets
    // from the block's first row; the layout's 4 GiB bound per (sequence, KV head) covers it.
    if ((static_cast<uint64_t>(kv->capacity) + 64u) * static_cast<uint64_t>(kv->pos_stride) * 2u >
        0xFFFFFF00ull)
        return GQA_ERR_INVALID_CONFIG;
    a = PrefillArgs{};
    a.k_new = k_new;
    a.v_new = v_new;
    a.k = k_cache;
    a.v = v_cache;
    a.start = start;
    a.kv_batch_stride = kv->batch_stride;
    a.kv_head_stride = kv->head_stride;
    a.kv_pos_stride = kv->pos_stride;
    a.capacity = kv->capacity;
    a.batch = batch;
    a.n_new = n_new;
    a.n_qblk = (n_new + 31) / 32;
    a.qk_scale_log2 = qk_scale_log2(params);
    a.flags = params->flags;
    fill_rope_table(params->rope_theta, &a.rope);
    return GQA_OK;
}

}  // namespace

extern "C" {

size_t gqa_prefill_workspace_bytes(const gqa_params_t* params, int32_t batch, int32_t n_new, int32_t capacity) {
    if (!params || !geometry_ok(params) || batch <= 0 || n_new <= 0 || capacity < n_new) return 0;
    // The multi-token path stages nothing: the chunk's unrounded keys enter through the
    // scores its preparation kernel forms, and the cache is read as stored.
    if (use_multi(params, n_new))
        return align_up(prefill_multi_bytes(batch, n_new, multi_wgs(params, n_new)), 256) +
               rescore_bytes(batch, n_new, 1, n_new, 0);
    return align_up(prefill_stage_bytes(batch, n_new, capacity), 256) +
           rescore_bytes(batch, n_new, prefill_chunk_blocks(n_new), 64, prefill_cache_blocks(capacity));
}

size_t gqa_prefill_rescored_rows_offset(const gqa_params_t* params, int32_t batch, int32_t n_new,
                                        int32_t capacity) {
    if (!gqa_prefill_workspace_bytes(params, batch, n_new, capacity)) return 0;
    // The rescore region (its first word: the flagged-row count) follows the path's own part.
    if (use_multi(params, n_new)) return align_up(prefill_multi_bytes(batch, n_new, multi_wgs(params, n_new)), 256);
    return align_up(prefill_stage_bytes(batch, n_new, capacity), 256);
}

int gqa_kv_append_bf16(const gqa_params_t* params, const uint16_t* k_new, const uint16_t* v_new,
                       uint16_t* k_cache, uint16_t* v_cache, const gqa_kv_layout_t* kv,
                       const int32_t* start, int32_t batch, int32_t n_new, void* stream) {
    PrefillArgs a;
    const int st = prefill_args(params, k_new, v_new, k_cache, v_cache, kv, start, batch, n_new, a);
    if (st != GQA_OK) return st;
    const hipError_t e = launch_kv_append(a, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GQA_OK : GQA_ERR_HIP;
}

int gqa_kv_append_paged_bf16(const gqa_params_t* params, const uint16_t* k_new, const uint16_t* v_new,
                             uint16_t* k_pool, uint16_t* v_pool, const gqa_paged_kv_t* kv,
                             const int32_t* block_table, const int32_t* start, int32_t batch, int32_t n_new,
                             void* stream) {
    if (!kv) return GQA_ERR_BAD_POINTER;
    if (!paged_layout_ok(kv)) return GQA_ERR_INVALID_CONFIG;
    if (!block_table) return GQA_ERR_BAD_POINTER;
    if (!aligned(block_table, 4)) return GQA_ERR_BAD_POINTER;
    gqa_kv_layout_t lay{kv->block_stride, kv->head_stride, kv->pos_stride, kv->max_blocks * 16};
    PrefillArgs a;
    const int st = prefill_args(params, k_new, v_new, k_pool, v_pool, &lay, start, batch, n_new, a);
    if (st != GQA_OK) return st;
    a.block_table = block_table;
    a.max_blocks = kv->max_blocks;
    a.n_blocks = kv->n_blocks;
    const hipError_t e = launch_kv_append(a, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? GQA_OK : GQA_ERR_HIP;
}

int gqa_prefill_bf16(const gqa_params_t* params, const uint16_t* q, const uint16_t* k_new,
                     const uint16_t* v_new, uint16_t* k_cache, uint16_t* v_cache,
                     const gqa_kv_layout_t* kv, const int32_t* start, int32_t batch, int32_t n_new,
                     uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
    PrefillArgs a;
    const int st = prefill_args(params, k_new, v_new, k_cache, v_cache, kv, start, batch, n_new, a);
    if (st != GQA_OK) return st;
    if (!q || !out) return GQA_ERR_BAD_POINTER;
    if (!aligned(q, 2) || !aligned(out, 8)) return GQA_ERR_BAD_POINTER;
    const size_t need = gqa_prefill_workspace_bytes(params, batch, n_new, kv->capacity);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256)) return GQA_ERR_WORKSPACE;
    a.q = q;
    a.out = out;
    const bool multi = use_multi(params, n_new);
    char* ws = static_cast<char*>(workspace);
    if (multi) {
        prefill_multi_layout(a, workspace, multi_wgs(params, n_new));
        a.skew_pm = xcd_skew_pm(multi_waves(n_new) == 1 ? 80 : multi_waves(n_new) == 2 ? 40 : 0);
        rescore_layout(a, params, ws + align_up(prefill_multi_bytes(batch, n_new, multi_wgs(params, n_new)), 256), 1,
                       n_new, 0);
    } else {
        prefill_stage_layout(a, workspace);
        rescore_layout(a, params, ws + align_up(prefill_stage_bytes(batch, n_new, kv->capacity), 256),
                       prefill_chunk_blocks(n_new), 64, prefill_cache_blocks(kv->capacity));
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipEvent_t* ev = profile_slot();
    if (ev) (void)hipEventRecord(ev[0], s);
    if (multi) {
        // The preparation kernel of the multi-token path appends the chunk's rows itself.
        hipError_t e = launch_prefill_multi(a, s, ev);
        if (e == hipSuccess) e = launch_rescore(a, s);
        if (ev) (void)hipEventRecord(ev[4], s);
        return e == hipSuccess ? GQA_OK : GQA_ERR_HIP;
    }
    // The attention kernel decides the rescore flag of each row it writes, from the K/V
    // statistics the staging and reduce kernels leave.
    hipError_t e = launch_kv_append(a, s);
    if (e == hipSuccess) e = launch_prefill_stage(a, s);
    if (e == hipSuccess) e = launch_prefill_stat_reduce(a, s);
    if (ev) (void)hipEventRecord(ev[1], s);
    if (e == hipSuccess) e = launch_prefill_attention(a, s);
    if (ev) (void)hipEventRecord(ev[2], s);
    if (e == hipSuccess) e = launch_rescore(a, s);
    if (ev) {
        (void)hipEventRecord(ev[3], s);
        (void)hipEventRecord(ev[4], s);
    }
    return e == hipSuccess ? GQA_OK : GQA_ERR_HIP;
}

}  // extern "C"

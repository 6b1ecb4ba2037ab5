// kvrt_runtime.hip — host side of the kvrt C ABI (include/kvrt.h).
//
// Owns the per-layer KV storage, the host-authoritative lengths and page
// tables, their device mirrors, and the split-K workspace. Validation happens
// before any enqueue; a failed enqueue poisons the context (no retry, no
// fallback), mirroring the fail-closed contract of the reference batch
// executor (native/gemma4_listener_microbatch/MICROBATCH_DESIGN.md:38-43).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <random>
#include <utility>
#include <vector>

#include "kvrt_internal.h"

using namespace kvrt;

// Scratch of kvrt_attend_tensors_noalloc_async: the split-K partials, mask
// records and error flag of one call, laid out as a per-stream workspace of
// kvrt_attend_tensors_async. Every GPU the library runs on holds its own copy
// until the process ends. In host code the name is not a device address:
// each device's copy is looked up once with hipGetSymbolAddress and only that
// pointer reaches the kernels.
constexpr size_t kScratchBytes = KVRT_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

struct Layer {
    kvrt_layer_spec spec{};
    int owner = 0;          // layer index whose storage and length this layer uses
    void *k = nullptr, *v = nullptr;
    float *ks = nullptr, *vs = nullptr;
    bool owned = false;
    uint64_t kv_bytes = 0, scale_bytes = 0;
    float *inv_freq = nullptr;  // device RoPE table [head_dim / 2] (kvrt_set_layer_rope)
    float rope_scaling = 1.f;
};

bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }
int ilog2(int x) { int s = 0; while ((1 << s) < x) ++s; return s; }

int elem_size(int dtype) {
    switch (dtype) {
        case KVRT_BF16: return 2;
        case KVRT_INT8: return 1;
        case KVRT_FP32: return 4;
        case KVRT_BOOL: return 1;
        case KVRT_INT32: return 4;
        case KVRT_INT64: return 8;
        default: return 0;
    }
}

// Host record of one slot: its generation (renewed when its contents are
// replaced) and the length of its prefix-attention mask.
struct SlotState {
    uint64_t generation = 0;
    int32_t prefix_len = 0;
};

int env_int(const char *name, int dflt) {
    const char *s = std::getenv(name);
    if (!s || !*s) return dflt;
    const int v = std::atoi(s);
    return v > 0 ? v : dflt;
}

}  // namespace

struct kvrt_ctx {
    kvrt_config cfg{};
    std::vector<Layer> layers;
    hipStream_t stream = nullptr;
    bool dirty = false;             // work enqueued since the bound stream was last synchronised
    bool lens_stale = false;        // work captured into a graph since the host lengths were read back
    int device = 0;
    bool poisoned = false;
    bool inject = false;
    std::vector<SlotState> slot;    // per slot
    uint64_t next_generation = 1;
    PrefixMask *d_prefix = nullptr; // device [n_slots] prefix-attention masks
    std::vector<int32_t> len;       // host shadow [slot * n_layers + layer]
    int32_t *d_len = nullptr;
    int32_t *d_err = nullptr;
    uint32_t *d_cnt = nullptr;      // arrival counters of single-launch decodes [kCntWords], zero between launches
    bool paged = false;
    int pt_stride = 0;
    std::vector<int32_t> pt;        // host page table mirror, -1 unmapped
    int32_t *d_pt = nullptr;
    std::vector<int32_t> free_pages;
    std::vector<int32_t> first_live; // per slot: first mapped logical page
    float *ws = nullptr;
    size_t ws_bytes = 0;
    std::vector<float *> retired_ws;  // kept until destroy: captured graphs may reference them
    LayerDesc *d_desc = nullptr;      // device [n_layers] layer descriptions
    kvrt_counters counters{};

    // RING layers, host only [slot * n_layers + layer]: the lowest position
    // whose row the ring still holds. An append raises it to length -
    // ring_rows; a rollback leaves it where it is, so a second rollback (or
    // one after a shorter re-append) cannot reach rows that positions past the
    // first rollback point overwrote.
    std::vector<int32_t> ring_lo;

    int len_at(int slot, int layer) const { return len[(size_t)slot * cfg.n_layers + layers[layer].owner]; }
    int &len_ref(int slot, int layer) { return len[(size_t)slot * cfg.n_layers + layers[layer].owner]; }
    int ring_floor(int slot, int layer) const { return ring_lo[(size_t)slot * cfg.n_layers + layers[layer].owner]; }
    // after the (slot, layer) length grew: rows below length - ring_rows are overwritten
    void ring_advance(int slot, int layer) {
        const Layer &o = layers[layers[layer].owner];
        if (o.spec.layout != KVRT_LAYOUT_RING) return;
        const size_t i = (size_t)slot * cfg.n_layers + layers[layer].owner;
        ring_lo[i] = std::max(ring_lo[i], len[i] - o.spec.ring_rows);
    }
    void ring_set(int slot, int layer, int lo) { ring_lo[(size_t)slot * cfg.n_layers + layers[layer].owner] = lo; }
};

namespace {

int poison(kvrt_ctx *c) {
    c->poisoned = true;
    return KVRT_EDEVICE;
}

int device_ok(kvrt_ctx *c, hipError_t e) {
    if (e != hipSuccess) return poison(c);
    return KVRT_OK;
}

// Preamble of every mutating call. A call refused by its argument checks
// enqueues nothing and leaves the context as it was (enq below marks work in
// flight).
int begin(kvrt_ctx *c) {
    if (!c) return KVRT_EINVAL;
    if (c->poisoned) return KVRT_EPOISONED;
    if (c->inject) {
        c->inject = false;
        return poison(c);
    }
    // Switch devices only when needed: hipSetDevice is refused inside a
    // stream capture, and calls of one context are captured into graphs.
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return poison(c);
    if (cur != c->device && hipSetDevice(c->device) != hipSuccess) return poison(c);
    return KVRT_OK;
}

// The bound stream, for an enqueue: the context counts as having work in
// flight on it from here until a synchronising call. Work enqueued while the
// stream is capturing only runs when the graph is replayed, which advances
// the device lengths behind the host's back: the host lengths stay
// unverified until kvrt_sync_lengths reads them back.
hipStream_t enq(kvrt_ctx *c) {
    c->dirty = true;
    if (!c->lens_stale) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        const hipError_t e = hipStreamIsCapturing(c->stream, &st);
        if (e != hipSuccess) (void)hipGetLastError();  // the launch that follows reports its own status
        if (e != hipSuccess || st != hipStreamCaptureStatusNone) c->lens_stale = true;
    }
    return c->stream;
}

KVView make_view(kvrt_ctx *c, int layer) {
    const Layer &L = c->layers[c->layers[layer].owner];
    const kvrt_layer_spec &s = L.spec;
    KVView v{};
    v.k = L.k;
    v.v = L.v;
    v.ks = L.ks;
    v.vs = L.vs;
    v.layout = s.layout;
    v.kv_heads = s.kv_heads;
    v.row_stride = s.head_dim;
    if (s.layout == KVRT_LAYOUT_CONTIG) {
        v.rows = c->cfg.capacity;
    } else if (s.layout == KVRT_LAYOUT_RING) {
        v.rows = s.ring_rows;
    } else {
        v.rows = c->cfg.block_size;
        v.block_shift = ilog2(c->cfg.block_size);
        v.page_table = c->d_pt;
        v.pt_stride = c->pt_stride;
        v.pool_pages = c->cfg.pool_pages;
    }
    v.head_stride = (int64_t)v.rows * s.head_dim;
    v.slot_stride = v.head_stride * s.kv_heads;
    return v;
}

// Upload the device layer descriptions (views, head dims, RoPE tables).
int upload_desc(kvrt_ctx *c) {
    std::vector<LayerDesc> h(c->cfg.n_layers);
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        const Layer &L = c->layers[c->layers[l].owner];
        h[l].kv = make_view(c, l);
        h[l].head_dim = L.spec.head_dim;
        h[l].dtype = L.spec.dtype;
        h[l].rope_scaling = L.rope_scaling;
        h[l].rope_pairs = L.inv_freq ? L.spec.head_dim / 2 : 0;
        h[l].inv_freq = L.inv_freq;
    }
    if (!c->d_desc && hipMalloc((void **)&c->d_desc, h.size() * sizeof(LayerDesc)) != hipSuccess)
        return KVRT_EDEVICE;
    if (hipMemcpy(c->d_desc, h.data(), h.size() * sizeof(LayerDesc), hipMemcpyHostToDevice) != hipSuccess)
        return KVRT_EDEVICE;
    return KVRT_OK;
}

Lengths make_len(kvrt_ctx *c, int layer) {
    Lengths l{};
    l.lens = c->d_len;
    l.stride = c->cfg.n_layers;
    l.offset = c->layers[layer].owner;
    return l;
}

bool valid_slot(const kvrt_ctx *c, int s) { return s >= 0 && s < c->cfg.n_slots; }
bool valid_layer(const kvrt_ctx *c, int l) { return l >= 0 && l < c->cfg.n_layers; }

bool distinct_slots(const kvrt_ctx *c, int n, const int32_t *slots) {
    if (n <= 0 || n > kMaxItems || !slots) return false;
    for (int i = 0; i < n; ++i) {
        if (!valid_slot(c, slots[i])) return false;
        for (int j = 0; j < i; ++j)
            if (slots[j] == slots[i]) return false;
    }
    return true;
}

// Tensor with the given dtype and rank; last dim contiguous; 16-byte aligned
// rows. Dims are checked by the callers.
bool tensor_ok(const kvrt_tensor *t, int dtype, int ndim) {
    if (!t || !t->data || t->dtype != dtype || t->ndim != ndim) return false;
    if (t->strides[ndim - 1] != 1) return false;
    const int es = elem_size(dtype);
    if ((reinterpret_cast<uintptr_t>(t->data) & 15u) != 0) return false;
    for (int i = 0; i < ndim - 1; ++i) {
        if (t->dims[i] > 1 && ((t->strides[i] * es) & 15) != 0) return false;
        if (t->strides[i] < 0) return false;
    }
    for (int i = 0; i < ndim; ++i)
        if (t->dims[i] < 0) return false;
    return true;
}

// tensor_ok, or an empty tensor of that dtype and rank (torch gives those a
// null data pointer); for calls that launch nothing when a dimension is 0.
bool tensor_ok_or_empty(const kvrt_tensor *t, int dtype, int ndim) {
    if (!t || t->dtype != dtype || t->ndim != ndim) return false;
    for (int i = 0; i < ndim; ++i)
        if (t->dims[i] < 0) return false;
    for (int i = 0; i < ndim; ++i)
        if (t->dims[i] == 0) return true;
    return tensor_ok(t, dtype, ndim);
}

bool is_contiguous(const kvrt_tensor *t) {
    int64_t expect = 1;
    for (int i = t->ndim - 1; i >= 0; --i) {
        if (t->dims[i] != 1 && t->strides[i] != expect) return false;
        expect *= t->dims[i];
    }
    return true;
}

constexpr int kMaxWgPerHead = 64;

// Which bf16 decodes run on the MFMA kernel (kvrt_config.decode_kernel).
// AUTO (bf16): 16 query rows per kv head (GQA group 8 with Q = 2), 8 rows at
// head_dim 512, 8 rows at head_dim <= 256 over at least kMfmaDecodeMinKeys8
// visible keys, and 1-4 rows over as many keys where the tiles stream through
// the LDS DMA ring (mfma_decode_dma) — the shapes where the VALU kernel's
// dot products and P.V products make it compute-bound. Short 8-row decodes (a
// 512-key sliding window) stay on the VALU kernel: latency-bound either way,
// and lighter on a concurrent stream. `keys` is the launch's key count
// rounded up to the split bucket, so the choice, like the split count, stays
// fixed within a bucket.
constexpr int64_t kMfmaDecodeMinKeys8 = 2048;
bool use_mfma_decode(int mode, int dtype, int rows_tile_, int head_dim, int64_t keys, int layout) {
    if (mode == KVRT_DECODE_VALU) return false;
    // int8 (PAGED): AUTO keeps the VALU kernel. A forced MFMA decode runs
    // the int8 ring kernel at head_dim 64 / 128 (i8_mfma_dma), the register-
    // staged MFMA tiles elsewhere. At config 5's layer the ring kernel runs
    // about as long as the VALU kernel (fused append + attend 31.7 vs 29.2
    // us) with a third of its VALU instructions, and the step slower (0.838
    // vs 0.808 ms when both quantised the new rows twice); KVRT_I8_MFMA=1
    // lets AUTO take it.
    if (dtype == KVRT_INT8) {
        static const char *env = std::getenv("KVRT_I8_MFMA");
        static const bool ring = env && std::atoi(env) != 0;
        return mode == KVRT_DECODE_MFMA || (ring && i8_mfma_dma(head_dim, rows_tile_));
    }
    if (rows_tile_ < kMfmaDecodeMinRows) {
        // 1-4 rows (the talker's 2) ride an 8-row tile: AUTO takes it where
        // the tiles stream through the LDS DMA ring, over as many keys as the
        // 8-row rule (talker launch 19.2 -> 17.8 us, step 0.565 -> 0.542 ms);
        // KVRT_MFMA_SMALL_ROWS=0 keeps them on the VALU kernel
        static const char *env = std::getenv("KVRT_MFMA_SMALL_ROWS");
        static const bool small = !env || std::atoi(env) != 0;
        static const int64_t min_keys_small = env_int("KVRT_MFMA_SMALL_MIN_KEYS", (int)kMfmaDecodeMinKeys8);
        return mode == KVRT_DECODE_MFMA ||
               (small && mfma_decode_dma(head_dim, rows_tile_, dtype, layout) && keys >= min_keys_small);
    }
    return mode == KVRT_DECODE_MFMA || rows_tile_ >= 16 || head_dim >= 512 || keys >= kMfmaDecodeMinKeys8;
}

// Split-K workgroups a decode launch aims at: the context's decode_wgs, else
// KVRT_TARGET_WGS (512), doubled for int8 layers — their VALU-bound waves
// (2 groups of 8 keys per pass, 118 VGPRs) need 4 waves per SIMD to hide the
// dequantise and FMA latencies.
int target_wgs(const kvrt_config &cfg, int dtype = KVRT_BF16) {
    static const int v = env_int("KVRT_TARGET_WGS", 512);
    if (cfg.decode_wgs > 0) return cfg.decode_wgs;
    return dtype == KVRT_INT8 ? 2 * v : v;
}
// Keys a wave must own at least: one main-loop iteration of the kernel
// variant (8..32 keys), unless KVRT_MIN_KEYS_PER_WAVE asks for more.
int min_keys_per_wave(int keys_per_iter) {
    static const int v = env_int("KVRT_MIN_KEYS_PER_WAVE", 1);
    return std::max(v, keys_per_iter);
}

// Number of wave splits per (item, kv head): enough workgroups to fill the
// chip, but at least min_keys keys per wave. n_items * kv_heads * (splits /
// kWaves) <= target + n_items * kv_heads, which bounds the workspace.
// The key count is rounded up to a multiple of kSplitKeyBucket, so that the
// split count, and with it the order of the fp32 reductions, stays the same
// over the decode steps of a bucket: a HIP graph captured at one length and
// replayed at the next ones then matches eager calls bit for bit.
#ifndef KVRT_SPLIT_KEY_BUCKET
#define KVRT_SPLIT_KEY_BUCKET 128
#endif
constexpr int64_t kSplitKeyBucket = KVRT_SPLIT_KEY_BUCKET;
// Whether a decode merges its workgroup partials in its last workgroup
// (kvrt_config.decode_merge) instead of a second kernel. AUTO: when the
// partials of one (item, kv head) total at most KVRT_SINGLE_LAUNCH_BYTES
// (32 KiB): the merging workgroup reads them all, three dependent memory
// round trips after the last partial lands, which costs about what the merge
// kernel's launch does; beyond that one workgroup's read takes longer.
bool single_launch_decode(int mode, bool mfma, int head_dim, int R, int rows, int n_parts) {
    static const int limit = env_int("KVRT_SINGLE_LAUNCH_BYTES", 32768);
    if (mode == KVRT_MERGE_SEPARATE || !(mfma || decode_wg_merge(head_dim, R))) return false;
    return mode == KVRT_MERGE_LAST_WG || (int64_t)n_parts * rows * head_dim * 4 <= limit;
}

int choose_splits(int target, int n_items, int kv_heads, int64_t max_keys, int keys_per_iter) {
    const int per_head = n_items * kv_heads;
    const int64_t per_wg = (int64_t)kWaves * min_keys_per_wave(keys_per_iter);
    int wg = (target + per_head - 1) / per_head;
    const int64_t bucket = (max_keys + kSplitKeyBucket - 1) / kSplitKeyBucket * kSplitKeyBucket;
    const int64_t cap = std::max<int64_t>(1, (bucket + per_wg - 1) / per_wg);
    if (wg > cap) wg = (int)cap;
    if (wg > kMaxWgPerHead) wg = kMaxWgPerHead;  // fix-up merges <= 256 wave partials
    if (wg < 1) wg = 1;
    return wg * kWaves;
}

// Split-K workspace bytes for n items of kv_heads heads, R rows, head dim D.
size_t workspace_bytes(int n_items, int kv_heads, int n_split, int R, int D) {
    const size_t parts = (size_t)n_items * kv_heads * n_split * R;
    return ((parts * D + 63) / 64) * 64 * 4 + parts * 8 + 256;
}

// Largest workspace any call on this context can need (max_q rows of up to
// 16 q heads per kv head -> R <= 16).
size_t workspace_bound(const kvrt_ctx *c) {
    const int n = std::min(c->cfg.n_slots, kMaxItems);
    size_t best = 0;
    for (const Layer &L : c->layers) {
        const int hkv = L.spec.kv_heads;
        const int total_wgs = std::min(target_wgs(c->cfg, L.spec.dtype) + n * hkv, n * hkv * kMaxWgPerHead);
        const size_t parts = (size_t)total_wgs * kWaves * 16;
        best = std::max(best, ((parts * L.spec.head_dim + 63) / 64) * 64 * 4 + parts * 8 + 256);
    }
    return best;
}

int ensure_workspace(kvrt_ctx *c, size_t bytes) {
    if (bytes <= c->ws_bytes) return KVRT_OK;
    // Never allocate inside a stream capture (the bound sized at create
    // covers every call, so this only triggers if the tuning changed).
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(c->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone)
        return KVRT_ESTATE;
    if (c->ws) {
        c->retired_ws.push_back(c->ws);  // a captured graph may still use it
        c->ws = nullptr;
        c->ws_bytes = 0;
    }
    size_t want = std::max(bytes, (size_t)1 << 20);
    if (hipMalloc(&c->ws, want) != hipSuccess) {
        c->ws = nullptr;
        return poison(c);
    }
    c->ws_bytes = want;
    return KVRT_OK;
}

int visible_keys(const kvrt_layer_spec &s, int len, int q) {
    if (s.window > 0) return std::min(len, s.window + q - 1);
    return len;
}

// Allocate pages for positions [from, to) of slot; records device edits.
int map_pages(kvrt_ctx *c, int slot, int from, int to, std::vector<int32_t> &idx,
              std::vector<int32_t> &val) {
    const int bs = c->cfg.block_size;
    if (to <= from) return KVRT_OK;
    const int p_lo = from / bs, p_hi = (to - 1) / bs;
    if (p_hi >= c->pt_stride) return KVRT_ESTATE;
    std::vector<std::pair<int, int>> taken;
    for (int p = p_lo; p <= p_hi; ++p) {
        int32_t &e = c->pt[(size_t)slot * c->pt_stride + p];
        if (e >= 0) continue;
        if (c->free_pages.empty()) {
            for (auto &t : taken) {  // roll back this call's allocations
                c->pt[(size_t)slot * c->pt_stride + t.first] = -1;
                c->free_pages.push_back(t.second);
                c->counters.pages_in_use--;
            }
            for (size_t i = 0; i < taken.size(); ++i) {
                idx.pop_back();
                val.pop_back();
            }
            return KVRT_ENOMEM;
        }
        const int page = c->free_pages.back();
        c->free_pages.pop_back();
        e = page;
        taken.push_back({p, page});
        idx.push_back(slot * c->pt_stride + p);
        val.push_back(page);
        c->counters.pages_in_use++;
    }
    return KVRT_OK;
}

// Undo page allocations recorded in (idx, val) that were not yet enqueued.
void unmap_pages(kvrt_ctx *c, const std::vector<int32_t> &idx, const std::vector<int32_t> &val) {
    for (size_t i = idx.size(); i-- > 0;) {
        c->pt[idx[i]] = -1;
        c->free_pages.push_back(val[i]);
        c->counters.pages_in_use--;
    }
}

// Map pages for [L_i, L_i + q) of every item; all-or-nothing.
int map_items(kvrt_ctx *c, int n, const int32_t *slots, const std::vector<int> &from, int q,
              std::vector<int32_t> &idx, std::vector<int32_t> &val) {
    for (int i = 0; i < n; ++i) {
        const int r = map_pages(c, slots[i], from[i], from[i] + q, idx, val);
        if (r != KVRT_OK) {
            unmap_pages(c, idx, val);
            idx.clear();
            val.clear();
            return r;
        }
    }
    return KVRT_OK;
}

int enqueue_pages(kvrt_ctx *c, const std::vector<int32_t> &idx, const std::vector<int32_t> &val) {
    if (idx.empty()) return KVRT_OK;
    c->counters.launches += (idx.size() + kPtUpdates - 1) / kPtUpdates;
    if (launch_set_pages(c->d_pt, (int)idx.size(), idx.data(), val.data(), enq(c)) != hipSuccess)
        return poison(c);
    return KVRT_OK;
}

// Mirror host lengths len[idx[i]] to the device. With expect (a rollback),
// the device edits only if it still holds expect[i] at every index (else it
// raises the context's error flag), so a rollback validated against stale
// host lengths never lands.
int set_device_lens(kvrt_ctx *c, const std::vector<int32_t> &idx, const std::vector<int32_t> *expect = nullptr) {
    for (size_t off = 0; off < idx.size(); off += kPtUpdates) {
        SetLenArgs a{};
        a.lens = c->d_len;
        a.n = (int)std::min<size_t>(kPtUpdates, idx.size() - off);
        a.check = expect != nullptr;
        a.err = c->d_err;
        for (int i = 0; i < a.n; ++i) {
            a.idx[i] = idx[off + i];
            a.val[i] = c->len[idx[off + i]];
            if (expect) a.expect[i] = (*expect)[off + i];
        }
        c->counters.launches++;
        if (launch_set_lens(a, enq(c)) != hipSuccess) return poison(c);
    }
    return KVRT_OK;
}

// The slot's contents were replaced: callers holding its old generation are stale.
void renew_generation(kvrt_ctx *c, int slot) { c->slot[slot].generation = c->next_generation++; }

bool generation_ok(const kvrt_ctx *c, int slot, uint64_t expected) {
    return expected == KVRT_ANY_GENERATION || c->slot[slot].generation == expected;
}

// Set the length word of a slot's device mask record (0 disables the mask).
int set_prefix_len_device(kvrt_ctx *c, int slot, int len) {
    SetLenArgs a{};
    a.lens = reinterpret_cast<int32_t *>(c->d_prefix);
    a.n = 1;
    a.idx[0] = slot * (int)(sizeof(PrefixMask) / sizeof(int32_t));
    a.val[0] = len;
    c->counters.launches++;
    if (launch_set_lens(a, enq(c)) != hipSuccess) return poison(c);
    c->slot[slot].prefix_len = len;
    return KVRT_OK;
}

// Device masks for a launch over these slots: the context's records when one
// of them has a mask, else null (the kernels then read no mask at all).
const PrefixMask *launch_masks(const kvrt_ctx *c, int n, const int32_t *slots) {
    for (int i = 0; i < n; ++i)
        if (c->slot[slots[i]].prefix_len > 0) return c->d_prefix;
    return nullptr;
}

// Validate a prefix-attention mask tensor of `items` rows ([items, P], or
// [P] / [1, P] for one row) and fill the pack arguments (except dst/index).
int prefix_tensor(const kvrt_tensor *m, int items, PrefixPackArgs &a) {
    if (!m || !m->data) return KVRT_EINVAL;
    const int es = elem_size(m->dtype);
    if (m->dtype != KVRT_INT64 && m->dtype != KVRT_INT32 && m->dtype != KVRT_BOOL) return KVRT_EINVAL;
    int64_t rows, plen, item_stride;
    if (m->ndim == 1 && items == 1) {
        rows = 1, plen = m->dims[0], item_stride = 0;
        if (plen > 1 && m->strides[0] != 1) return KVRT_EINVAL;
    } else if (m->ndim == 2) {
        rows = m->dims[0], plen = m->dims[1], item_stride = m->strides[0];
        if (plen > 1 && m->strides[1] != 1) return KVRT_EINVAL;
    } else {
        return KVRT_EINVAL;
    }
    if (rows != items || plen < 0 || plen > KVRT_MAX_PREFIX_MASK || item_stride < 0) return KVRT_EINVAL;
    if ((reinterpret_cast<uintptr_t>(m->data) % (uintptr_t)es) != 0) return KVRT_EINVAL;
    a.src = static_cast<const uint8_t *>(m->data);
    a.item_stride = item_stride;
    a.elem_bytes = es;
    a.n_items = items;
    a.plen = (int)plen;
    return KVRT_OK;
}

int create_impl(const kvrt_config *cfg, const kvrt_layer_spec *specs, const kvrt_storage *storage,
                kvrt_ctx **out) {
    if (!cfg || !specs || !out) return KVRT_EINVAL;
    *out = nullptr;
    if (cfg->struct_size != sizeof(kvrt_config)) return KVRT_EINVAL;
    if (cfg->n_layers <= 0 || cfg->n_layers > 4096 || cfg->n_slots <= 0 || cfg->n_slots > (1 << 20) ||
        cfg->capacity <= 0 || cfg->max_q <= 0 || cfg->max_q > 65536 || cfg->decode_wgs < 0 ||
        cfg->decode_wgs > 65536 || cfg->decode_kernel < KVRT_DECODE_AUTO || cfg->decode_kernel > KVRT_DECODE_MFMA ||
        cfg->decode_merge < KVRT_MERGE_AUTO || cfg->decode_merge > KVRT_MERGE_LAST_WG)
        return KVRT_EINVAL;
    bool any_paged = false;
    for (int i = 0; i < cfg->n_layers; ++i) {
        const kvrt_layer_spec &s = specs[i];
        if (s.shared_src >= 0) {
            if (s.shared_src >= i || specs[s.shared_src].shared_src >= 0) return KVRT_EINVAL;
            continue;
        }
        if (s.shared_src != -1) return KVRT_EINVAL;
        if (s.head_dim != 64 && s.head_dim != 128 && s.head_dim != 256 && s.head_dim != 512) return KVRT_EINVAL;
        if (s.kv_heads <= 0 || s.kv_heads > 64 || s.window < 0) return KVRT_EINVAL;
        if (s.dtype != KVRT_BF16 && s.dtype != KVRT_INT8) return KVRT_EINVAL;
        if (s.dtype == KVRT_INT8 && s.layout != KVRT_LAYOUT_PAGED) return KVRT_EINVAL;
        if (s.layout == KVRT_LAYOUT_RING) {
            if (s.window <= 0 || s.ring_rows < s.window + cfg->max_q - 1) return KVRT_EINVAL;
        } else if (s.layout == KVRT_LAYOUT_PAGED) {
            any_paged = true;
        } else if (s.layout != KVRT_LAYOUT_CONTIG) {
            return KVRT_EINVAL;
        }
    }
    if (any_paged && (!is_pow2(cfg->block_size) || cfg->block_size > 1024 || cfg->pool_pages <= 0 ||
                      cfg->pool_pages >= (1 << 24)))
        return KVRT_EINVAL;
    for (int i = 0; i < cfg->n_layers; ++i) {
        // the kernels number a pool's rows in 32 bits
        const kvrt_layer_spec &s = specs[i];
        if (s.shared_src < 0 && s.layout == KVRT_LAYOUT_PAGED && (int64_t)cfg->pool_pages * s.kv_heads * cfg->block_size > INT32_MAX)
            return KVRT_EINVAL;
    }

    kvrt_ctx *c = new (std::nothrow) kvrt_ctx();
    if (!c) return KVRT_EDEVICE;
    c->cfg = *cfg;
    if (hipGetDevice(&c->device) != hipSuccess) {
        delete c;
        return KVRT_EDEVICE;
    }
    c->layers.resize(cfg->n_layers);
    c->len.assign((size_t)cfg->n_slots * cfg->n_layers, 0);
    c->ring_lo.assign((size_t)cfg->n_slots * cfg->n_layers, 0);
    c->paged = any_paged;
    auto fail = [&](int code) {
        kvrt_destroy(c);
        return code;
    };
    for (int i = 0; i < cfg->n_layers; ++i) {
        Layer &L = c->layers[i];
        L.spec = specs[i];
        L.owner = specs[i].shared_src >= 0 ? specs[i].shared_src : i;
        if (specs[i].shared_src >= 0) L.spec = specs[specs[i].shared_src], L.spec.shared_src = specs[i].shared_src;
        if (specs[i].shared_src >= 0) continue;
        if (kvrt_layer_storage_bytes(cfg, &specs[i], &L.kv_bytes, &L.scale_bytes) != KVRT_OK) return fail(KVRT_EINVAL);
        if (storage) {
            const kvrt_storage &st = storage[i];
            if (!st.k || !st.v || (L.scale_bytes && (!st.k_scale || !st.v_scale))) return fail(KVRT_EINVAL);
            if (((reinterpret_cast<uintptr_t>(st.k) | reinterpret_cast<uintptr_t>(st.v) |
                  reinterpret_cast<uintptr_t>(st.k_scale) | reinterpret_cast<uintptr_t>(st.v_scale)) & 15u) != 0)
                return fail(KVRT_EINVAL);  // 16-byte rows and fills need aligned storage
            L.k = st.k;
            L.v = st.v;
            L.ks = static_cast<float *>(st.k_scale);
            L.vs = static_cast<float *>(st.v_scale);
            L.owned = false;
        } else {
            L.owned = true;
            if (hipMalloc(&L.k, L.kv_bytes) != hipSuccess || hipMalloc(&L.v, L.kv_bytes) != hipSuccess)
                return fail(KVRT_EDEVICE);
            if (L.scale_bytes) {
                if (hipMalloc((void **)&L.ks, L.scale_bytes) != hipSuccess ||
                    hipMalloc((void **)&L.vs, L.scale_bytes) != hipSuccess)
                    return fail(KVRT_EDEVICE);
            }
            if (launch_zero(L.k, L.kv_bytes, nullptr) != hipSuccess ||
                launch_zero(L.v, L.kv_bytes, nullptr) != hipSuccess)
                return fail(KVRT_EDEVICE);
            if (L.scale_bytes && (launch_zero(L.ks, L.scale_bytes, nullptr) != hipSuccess ||
                                  launch_zero(L.vs, L.scale_bytes, nullptr) != hipSuccess))
                return fail(KVRT_EDEVICE);
        }
    }
    const size_t len_bytes = ((c->len.size() * 4 + 15) / 16) * 16;
    if (hipMalloc((void **)&c->d_len, len_bytes) != hipSuccess) return fail(KVRT_EDEVICE);
    if (launch_zero(c->d_len, len_bytes, nullptr) != hipSuccess) return fail(KVRT_EDEVICE);
    if (hipMalloc((void **)&c->d_err, 16) != hipSuccess) return fail(KVRT_EDEVICE);
    if (launch_zero(c->d_err, 16, nullptr) != hipSuccess) return fail(KVRT_EDEVICE);
    if (hipMalloc((void **)&c->d_cnt, kCntWords * 4) != hipSuccess) return fail(KVRT_EDEVICE);
    if (launch_zero(c->d_cnt, kCntWords * 4, nullptr) != hipSuccess) return fail(KVRT_EDEVICE);
    const size_t prefix_bytes = (size_t)cfg->n_slots * sizeof(PrefixMask);
    if (hipMalloc((void **)&c->d_prefix, prefix_bytes) != hipSuccess) return fail(KVRT_EDEVICE);
    if (launch_zero(c->d_prefix, prefix_bytes, nullptr) != hipSuccess) return fail(KVRT_EDEVICE);
    c->slot.assign(cfg->n_slots, SlotState{});
    for (int i = 0; i < cfg->n_slots; ++i) renew_generation(c, i);
    if (any_paged) {
        c->pt_stride = (cfg->capacity + cfg->block_size - 1) / cfg->block_size;
        c->pt.assign((size_t)cfg->n_slots * c->pt_stride, -1);
        const size_t pt_bytes = ((c->pt.size() * 4 + 15) / 16) * 16;
        if (hipMalloc((void **)&c->d_pt, pt_bytes) != hipSuccess) return fail(KVRT_EDEVICE);
        if (hipMemcpy(c->d_pt, c->pt.data(), c->pt.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return fail(KVRT_EDEVICE);
        c->free_pages.reserve(cfg->pool_pages);
        for (int p = cfg->pool_pages - 1; p >= 0; --p) c->free_pages.push_back(p);
        if (cfg->pool_seed != 0) {
            std::mt19937 rng((uint32_t)cfg->pool_seed);
            std::shuffle(c->free_pages.begin(), c->free_pages.end(), rng);
        }
        c->first_live.assign(cfg->n_slots, 0);
    }
    c->ws_bytes = 0;
    if (ensure_workspace(c, workspace_bound(c)) != KVRT_OK) return fail(KVRT_EDEVICE);
    if (upload_desc(c) != KVRT_OK) return fail(KVRT_EDEVICE);
    if (hipDeviceSynchronize() != hipSuccess) return fail(KVRT_EDEVICE);
    *out = c;
    return KVRT_OK;
}

// bf16 round-to-nearest-even of a finite float, back as a float.
float round_bf16(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    std::memcpy(&x, &u, 4);
    return x;
}

// Validate the talker visibility of n items against the host lengths and
// lower it to the kernel's form; the key count of item i is audio_position + 1.
int talker_items(kvrt_ctx *c, int layer, int n, const int32_t *slots, const kvrt_talker_mask *m,
                 TalkerItem *out) {
    for (int i = 0; i < n; ++i) {
        const kvrt_talker_mask &t = m[i];
        if (t.prefix_attention_mode < 0 || t.prefix_attention_mode > 2 || !std::isfinite(t.prefix_log_gate) ||
            (t.prefix_attention_mode == 2 && t.visible_prefix_count <= 0))
            return KVRT_EINVAL;
        if (t.prefix_start < 0 || t.prefix_position < t.prefix_start || t.audio_start <= t.prefix_position ||
            t.audio_position < t.audio_start)
            return KVRT_EINVAL;
        if (t.audio_position >= c->len_at(slots[i], layer)) return KVRT_ESTATE;
        // the additive mask value of the reference: fp32 gate - logf(count), stored as bf16
        float g = 0.f;
        if (t.prefix_attention_mode == 2) {
            g = round_bf16(t.prefix_log_gate - logf((float)t.visible_prefix_count));
            if (!std::isfinite(g)) return KVRT_EINVAL;
        }
        out[i] = TalkerItem{t.prefix_start, t.prefix_position, t.audio_start, t.audio_position,
                            t.prefix_attention_mode, g * 1.4426950408889634f};
    }
    return KVRT_OK;
}

// Launch the split-K decode for n slots of one layer (fused when k/v given;
// under the talker visibility when masks is given).
int decode_impl(kvrt_ctx *c, int layer, int n, const int32_t *slots, const kvrt_tensor *q,
                const kvrt_tensor *k, const kvrt_tensor *v, const kvrt_tensor *out, float scale,
                const kvrt_talker_mask *masks = nullptr) {
    const kvrt_layer_spec &s = c->layers[layer].spec;
    const bool fused = k != nullptr;
    const bool talker = masks != nullptr;
    const int D = s.head_dim, hkv = s.kv_heads;
    if (!tensor_ok(q, KVRT_BF16, 4) || !tensor_ok(out, KVRT_BF16, 4) || !is_contiguous(q) || !is_contiguous(out))
        return KVRT_EINVAL;
    const int64_t hq = q->dims[1], qn = q->dims[2];
    if (q->dims[0] != n || q->dims[3] != D || hq <= 0 || hq % hkv != 0 || qn <= 0 || qn > c->cfg.max_q)
        return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (out->dims[i] != q->dims[i]) return KVRT_EINVAL;
    const int group = (int)(hq / hkv);
    const int rows = group * (int)qn;
    if (rows_tile(rows) == 0) return KVRT_EINVAL;
    if (s.dtype == KVRT_INT8 && rows_tile(rows) > kMaxInt8Rows) return KVRT_EINVAL;
    if (!std::isfinite(scale)) return KVRT_EINVAL;
    TalkerItem titems[kMaxItems];
    if (talker) {
        if (fused || s.dtype != KVRT_BF16 || s.layout != KVRT_LAYOUT_CONTIG || s.window != 0 || qn > 2)
            return KVRT_EINVAL;
        const int rc = talker_items(c, layer, n, slots, masks, titems);
        if (rc != KVRT_OK) return rc;
    }
    if (fused) {
        // int8 rows are quantised in-kernel by the VALU decode and the int8
        // MFMA ring kernel (the caller routes other forced MFMA decodes
        // through the append kernel)
        if (s.dtype == KVRT_INT8 && (s.layout != KVRT_LAYOUT_PAGED || (c->cfg.decode_kernel == KVRT_DECODE_MFMA &&
                                                                      !i8_mfma_dma(D, rows_tile(rows)))))
            return KVRT_EINVAL;
        if (!tensor_ok(k, KVRT_BF16, 4) || !tensor_ok(v, KVRT_BF16, 4) || !is_contiguous(k) || !is_contiguous(v))
            return KVRT_EINVAL;
        if (k->dims[0] != n || k->dims[1] != hkv || k->dims[2] != qn || k->dims[3] != D) return KVRT_EINVAL;
        for (int i = 0; i < 4; ++i)
            if (v->dims[i] != k->dims[i]) return KVRT_EINVAL;
    }
    // host-side state checks
    int64_t max_keys = 0;
    std::vector<int> from(n);
    std::vector<int64_t> item_keys(n);
    for (int i = 0; i < n; ++i) {
        const int L = c->len_at(slots[i], layer);
        const int Lnew = fused ? L + (int)qn : L;
        from[i] = L;
        if (Lnew < qn) return KVRT_ESTATE;
        if (fused && Lnew > c->cfg.capacity) return KVRT_ESTATE;
        // the oldest key any query of the call sees must be on a live page
        // (PAGED) or still in the ring (RING, after a rollback)
        const int oldest = s.window > 0 ? std::max(0, Lnew - (int)qn - s.window + 1) : 0;
        if (s.layout == KVRT_LAYOUT_PAGED && oldest < c->first_live[slots[i]] * c->cfg.block_size) return KVRT_ESTATE;
        if (s.layout == KVRT_LAYOUT_RING && oldest < c->ring_floor(slots[i], layer)) return KVRT_ESTATE;
        item_keys[i] = talker ? titems[i].audio_pos + 1 : visible_keys(s, Lnew, (int)qn);
        max_keys = std::max<int64_t>(max_keys, item_keys[i]);
    }
    const int R = rows_tile(rows);
    const int64_t bucket_keys = (max_keys + kSplitKeyBucket - 1) / kSplitKeyBucket * kSplitKeyBucket;
    const PrefixMask *pmask = talker ? nullptr : launch_masks(c, n, slots);
    // the MFMA kernel's PAGED D 512 variant has no registers for a mask
    const bool mfma = !talker && use_mfma_decode(c->cfg.decode_kernel, s.dtype, R, D, bucket_keys, s.layout) &&
                      !(pmask && s.layout == KVRT_LAYOUT_PAGED && D >= 512);
    const int mfma_keys = s.dtype == KVRT_INT8 && i8_mfma_dma(D, R) ? kI8MfmaKeys : kMfmaDecodeKeys;
    const int n_split = choose_splits(target_wgs(c->cfg, mfma ? KVRT_BF16 : s.dtype), n, hkv, max_keys,
                                      mfma ? mfma_keys : keys_per_iteration(D, R, s.dtype, s.layout));
    const int Rw = mfma ? std::max(R, kMfmaDecodeMinRows) : R;  // rows per partial (MFMA tiles are 8 or 16)
    const size_t acc_elems = (size_t)n * hkv * n_split * Rw * D;
    int rc = ensure_workspace(c, workspace_bytes(n, hkv, n_split, Rw, D));
    if (rc != KVRT_OK) return rc;
    std::vector<int32_t> pidx, pval;
    if (fused && s.layout == KVRT_LAYOUT_PAGED) {
        rc = map_items(c, n, slots, from, (int)qn, pidx, pval);
        if (rc != KVRT_OK) return rc;
    }
    DecodeArgs a{};
    if (pidx.size() <= (size_t)kMaxItems) {
        // the new rows' pages travel in the launch (its first workgroup
        // writes them into the table): no page-table launch ahead of it
        a.n_upd = (int)pidx.size();
        for (size_t i = 0; i < pidx.size(); ++i) {
            a.upd_idx[i] = pidx[i];
            a.upd_val[i] = pval[i];
        }
    } else {
        rc = enqueue_pages(c, pidx, pval);
        if (rc != KVRT_OK) return rc;
    }
    a.kv = make_view(c, layer);
    a.len = make_len(c, layer);
    a.q = static_cast<const uint16_t *>(q->data);
    a.out = static_cast<uint16_t *>(out->data);
    a.k_new = fused ? static_cast<const uint16_t *>(k->data) : nullptr;
    a.v_new = fused ? static_cast<const uint16_t *>(v->data) : nullptr;
    a.part_acc = c->ws;
    a.part_ml = reinterpret_cast<float2 *>(c->ws + ((acc_elems + 63) / 64) * 64);
    a.err = c->d_err;
    a.n_items = n;
    a.group = group;
    a.qn = (int)qn;
    a.window = s.window;
    a.n_split = n_split;
    a.advance = fused ? 1 : 0;
    a.n_parts = (mfma || decode_wg_merge(D, R)) ? n_split / kWaves : n_split;
    a.cnt = single_launch_decode(c->cfg.decode_merge, mfma, D, R, rows, a.n_parts) ? c->d_cnt : nullptr;
    a.pmask = pmask;
    a.scale_log2 = scale * 1.4426950408889634f;
    for (int i = 0; i < n; ++i) a.slots[i] = slots[i];
    // grid z order: most visible keys first (stable), so that a ragged batch's
    // longest workgroups start first
    std::vector<int> ord(n);
    for (int i = 0; i < n; ++i) ord[i] = i;
    std::stable_sort(ord.begin(), ord.end(), [&](int x, int y) { return item_keys[x] > item_keys[y]; });
    for (int i = 0; i < n; ++i) a.order[i] = (uint8_t)ord[i];
    c->counters.launches += a.cnt ? 1 : 2;
    c->counters.mfma_decodes += mfma ? 1 : 0;
    if (talker) {
        TalkerArgs t{};
        static_cast<DecodeArgs &>(t) = a;
        for (int i = 0; i < n; ++i) t.talk[i] = titems[i];
        if (launch_decode_talker(t, D, rows, enq(c)) != hipSuccess) return poison(c);
        for (int i = 0; i < n; ++i) {
            const uint64_t keys = (uint64_t)titems[i].audio_pos + 1;
            c->counters.attended_keys += keys * hkv;
            c->counters.attended_bytes += keys * hkv * (uint64_t)D * 2 * 2;
        }
        return KVRT_OK;
    }
    if ((mfma ? launch_decode_mfma(a, D, s.dtype, rows, enq(c)) : launch_decode(a, D, s.dtype, rows, enq(c))) !=
        hipSuccess)
        return poison(c);
    const int kb = s.dtype == KVRT_INT8 ? 1 : 2;
    for (int i = 0; i < n; ++i) {
        int &L = c->len_ref(slots[i], layer);
        if (fused) {
            L += (int)qn;
            c->ring_advance(slots[i], layer);
            c->counters.appended_rows += (uint64_t)qn * hkv;
            c->counters.appended_bytes += (uint64_t)qn * hkv * D * 2 * kb;
        }
        const uint64_t keys = (uint64_t)visible_keys(s, L, (int)qn);
        c->counters.attended_keys += keys * hkv;
        c->counters.attended_bytes += keys * hkv * (uint64_t)D * 2 * kb;
    }
    return KVRT_OK;
}

int append_impl(kvrt_ctx *c, int layer, int n, const int32_t *slots, const kvrt_tensor *k,
                const kvrt_tensor *v) {
    const kvrt_layer_spec &s = c->layers[layer].spec;
    if (c->layers[layer].owner != layer) return KVRT_OK;  // shared layers own no rows
    const int D = s.head_dim, hkv = s.kv_heads;
    if (!tensor_ok(k, KVRT_BF16, 4) || !tensor_ok(v, KVRT_BF16, 4)) return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (k->dims[i] != v->dims[i] || k->strides[i] != v->strides[i]) return KVRT_EINVAL;
    const int64_t qn = k->dims[2];
    if (k->dims[0] != n || k->dims[1] != hkv || k->dims[3] != D || qn <= 0 || qn > c->cfg.capacity)
        return KVRT_EINVAL;
    // Up to max_q rows: the device cursor picks the position (graph-replay
    // safe). Longer appends (prefill) take the host position, one item per
    // launch, and spread over many workgroups.
    if (qn > c->cfg.max_q && n > 1) {
        for (int i = 0; i < n; ++i) {
            kvrt_tensor ki = *k, vi = *v;
            ki.dims[0] = vi.dims[0] = 1;
            ki.data = static_cast<uint16_t *>(k->data) + i * k->strides[0];
            vi.data = static_cast<uint16_t *>(v->data) + i * v->strides[0];
            const int rc = append_impl(c, layer, 1, slots + i, &ki, &vi);
            if (rc != KVRT_OK) return rc;
        }
        return KVRT_OK;
    }
    std::vector<int> from(n);
    for (int i = 0; i < n; ++i) {
        from[i] = c->len_at(slots[i], layer);
        if ((int64_t)from[i] + qn > c->cfg.capacity) return KVRT_ESTATE;
    }
    std::vector<int32_t> pidx, pval;
    if (s.layout == KVRT_LAYOUT_PAGED) {
        const int r = map_items(c, n, slots, from, (int)qn, pidx, pval);
        if (r != KVRT_OK) return r;
        if ((int)pidx.size() > kPtUpdates) {  // too many edits for the kernarg block
            const int rc = enqueue_pages(c, pidx, pval);
            if (rc != KVRT_OK) return rc;
            pidx.clear();
            pval.clear();
        }
    }
    AppendArgs a{};
    a.kv = make_view(c, layer);
    a.len = make_len(c, layer);
    a.k_src = static_cast<const uint16_t *>(k->data);
    a.v_src = static_cast<const uint16_t *>(v->data);
    a.src_item_stride = k->strides[0];
    a.src_head_stride = k->strides[1];
    a.src_row_stride = k->strides[2];
    a.n_items = n;
    a.rows = (int)qn;
    a.import_mode = 0;
    a.err = c->d_err;
    a.n_upd = (int)pidx.size();
    for (size_t i = 0; i < pidx.size(); ++i) {
        a.upd_idx[i] = pidx[i];
        a.upd_val[i] = pval[i];
    }
    for (int i = 0; i < n; ++i) a.slots[i] = slots[i];
    int grid_x = 1;
    if (qn > c->cfg.max_q) {  // n == 1 here
        a.import_mode = 1;
        a.base_pos = from[0];
        // a ring keeps only its last ring_rows positions
        a.keep_from = s.layout == KVRT_LAYOUT_RING ? from[0] + (int)qn - s.ring_rows : 0;
        const int64_t chunks = (int64_t)hkv * qn * (D / 8);
        grid_x = (int)std::max<int64_t>(1, std::min<int64_t>(4096, (chunks + 255) / 256));
    }
    c->counters.launches++;
    if (launch_append(a, D, s.dtype, grid_x, enq(c)) != hipSuccess) return poison(c);
    const int kb = s.dtype == KVRT_INT8 ? 1 : 2;
    for (int i = 0; i < n; ++i) {
        c->len_ref(slots[i], layer) += (int)qn;
        c->ring_advance(slots[i], layer);
        c->counters.appended_rows += (uint64_t)qn * hkv;
        c->counters.appended_bytes += (uint64_t)qn * hkv * D * 2 * kb;
    }
    return KVRT_OK;
}

// Workspace of the context-free tensor attention, one per (device, stream):
// calls on one stream share it in stream order, calls on different streams
// never do. Layout: the error flag (kTensorWsHead floats), the prefix masks
// of the call's items (kMaxItems records), the arrival counters of
// single-launch decodes (zero between launches), then the split-K partials.
constexpr size_t kTensorWsHead = 64;
constexpr size_t kTensorWsMasks = kMaxItems * sizeof(PrefixMask) / sizeof(float);
constexpr size_t kTensorWsCnt = (kCntItemBase + kMaxItems + 63) / 64 * 64;
constexpr size_t kTensorWsParts = kTensorWsHead + kTensorWsMasks + kTensorWsCnt;

struct TensorWorkspace {
    float *ptr = nullptr;
    size_t bytes = 0;
};
// One lock for the map and for each call's launches: a decode and its merge
// kernel are enqueued together, so two host threads on one stream cannot
// interleave their partials.
std::mutex g_tensor_mu;
std::map<std::pair<int, hipStream_t>, TensorWorkspace> g_tensor_ws;
// Outgrown workspaces: never freed, since a captured graph may still use them.
std::vector<float *> g_tensor_retired;

// One context-free tensor attention call, validated and laid out: the decode
// arguments (workspace pointers unset), the prefix masks to pack, and the
// workspace bytes it needs.
struct TensorCall {
    DecodeArgs a{};
    PrefixPackArgs pk{};
    bool masked = false;
    bool mfma = false;
    bool single = false;  // the decode may merge its own partials (bit-identical to the merge kernel)
    int D = 0, rows = 0;
    size_t acc_elems = 0;
    size_t bytes = 0;
};

int tensor_call_setup(const kvrt_tensor *q, const kvrt_tensor *k, const kvrt_tensor *v, const int32_t *device_lengths,
                      const kvrt_tensor *prefix_attention, const kvrt_tensor *out, float scale, int32_t window,
                      int target, TensorCall &tc) {
    if (!device_lengths || window < 0 || !std::isfinite(scale)) return KVRT_EINVAL;
    if (!tensor_ok(q, KVRT_BF16, 4) || !tensor_ok(out, KVRT_BF16, 4) || !is_contiguous(q) || !is_contiguous(out))
        return KVRT_EINVAL;
    if (!tensor_ok(k, KVRT_BF16, 4) || !tensor_ok(v, KVRT_BF16, 4)) return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (k->dims[i] != v->dims[i] || k->strides[i] != v->strides[i] || out->dims[i] != q->dims[i])
            return KVRT_EINVAL;
    const int64_t n = q->dims[0], hq = q->dims[1], qn = q->dims[2], D = q->dims[3];
    const int64_t hkv = k->dims[1], lmax = k->dims[2];
    if (n <= 0 || n > kMaxItems || k->dims[0] != n || k->dims[3] != D || hkv <= 0 || hkv > 64 || hq % hkv != 0 ||
        qn <= 0 || qn > 64)
        return KVRT_EINVAL;
    if (D != 64 && D != 128 && D != 256 && D != 512) return KVRT_EINVAL;
    if (k->strides[2] != D) return KVRT_EINVAL;
    const int group = (int)(hq / hkv);
    const int rows = group * (int)qn;
    if (rows_tile(rows) == 0) return KVRT_EINVAL;
    if (prefix_attention != nullptr) {
        const int rc = prefix_tensor(prefix_attention, (int)n, tc.pk);
        if (rc != KVRT_OK) return rc;
        tc.masked = tc.pk.plen > 0;
    }
    DecodeArgs &a = tc.a;
    a.kv.k = k->data;
    a.kv.v = v->data;
    a.kv.layout = KVRT_LAYOUT_CONTIG;
    a.kv.kv_heads = (int)hkv;
    a.kv.rows = (int)lmax;
    a.kv.slot_stride = k->strides[0];
    a.kv.head_stride = k->strides[1];
    a.kv.row_stride = k->strides[2];
    a.len.lens = const_cast<int32_t *>(device_lengths);
    a.len.stride = 1;
    a.len.offset = 0;
    a.q = static_cast<const uint16_t *>(q->data);
    a.out = static_cast<uint16_t *>(out->data);
    a.n_items = (int)n;
    a.group = group;
    a.qn = (int)qn;
    a.window = window;
    const int R = rows_tile(rows);
    const int64_t keys = window > 0 ? std::min<int64_t>(lmax, window + qn - 1) : lmax;
    tc.mfma = use_mfma_decode(KVRT_DECODE_AUTO, KVRT_BF16, R, (int)D,
                              (keys + kSplitKeyBucket - 1) / kSplitKeyBucket * kSplitKeyBucket, KVRT_LAYOUT_CONTIG);
    a.n_split = choose_splits(target, (int)n, (int)hkv, keys,
                              tc.mfma ? kMfmaDecodeKeys : keys_per_iteration((int)D, R, KVRT_BF16, KVRT_LAYOUT_CONTIG));
    a.n_parts = (tc.mfma || decode_wg_merge((int)D, R)) ? a.n_split / kWaves : a.n_split;
    a.scale_log2 = scale * 1.4426950408889634f;
    for (int i = 0; i < n; ++i) a.order[i] = (uint8_t)i;
    for (int i = 0; i < n; ++i) a.slots[i] = i;
    const int Rw = tc.mfma ? std::max(R, kMfmaDecodeMinRows) : R;  // rows per partial
    tc.D = (int)D;
    tc.rows = rows;
    tc.acc_elems = (size_t)n * hkv * a.n_split * Rw * D;
    tc.bytes = (kTensorWsParts + tc.acc_elems + 64) * 4 + (size_t)n * hkv * a.n_split * Rw * 8;
    // At most 16 partials per (item, kv head): the last workgroup's merge
    // rounds exactly as the merge kernel's, so the result does not depend on
    // which of the two ran.
    tc.single = a.n_parts <= 16 && single_launch_decode(KVRT_MERGE_AUTO, tc.mfma, (int)D, R, rows, a.n_parts);
    return KVRT_OK;
}

// Device address of the scratch array on device dev (the current device),
// looked up on the device's first call and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

int scratch_pointer(int dev, float **out) {
    if (dev < 0 || dev >= kMaxDevices) return KVRT_EDEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return KVRT_EDEVICE;
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<float *>(g_scratch_ptr[dev]);
    return KVRT_OK;
}

// Enqueue a set-up call on workspace ws (at least tc.bytes, laid out as the
// per-stream workspaces: error flag, masks, partials).
int tensor_call_launch(TensorCall &tc, float *ws, hipStream_t st, bool single) {
    DecodeArgs &a = tc.a;
    a.err = reinterpret_cast<int32_t *>(ws);
    a.cnt = single && tc.single ? reinterpret_cast<uint32_t *>(ws + kTensorWsHead + kTensorWsMasks) : nullptr;
    a.part_acc = ws + kTensorWsParts;
    a.part_ml = reinterpret_cast<float2 *>(a.part_acc + ((tc.acc_elems + 63) / 64) * 64);
    if (tc.masked) {
        tc.pk.dst = reinterpret_cast<PrefixMask *>(ws + kTensorWsHead);
        for (int i = 0; i < a.n_items; ++i) tc.pk.index[i] = i;
        if (launch_prefix_pack(tc.pk, st) != hipSuccess) return KVRT_EDEVICE;
        a.pmask = tc.pk.dst;
    }
    if ((tc.mfma ? launch_decode_mfma(a, tc.D, KVRT_BF16, tc.rows, st) : launch_decode(a, tc.D, KVRT_BF16, tc.rows, st)) !=
        hipSuccess)
        return KVRT_EDEVICE;
    return KVRT_OK;
}

}  // namespace

// ===========================================================================
extern "C" {

uint32_t kvrt_abi_version(void) { return KVRT_ABI_VERSION; }

uint64_t kvrt_capabilities(void) {
    return KVRT_CAP_CONTIG | KVRT_CAP_RING | KVRT_CAP_PAGED | KVRT_CAP_INT8 | KVRT_CAP_FUSED_APPEND_ATTEND |
           KVRT_CAP_GATHER | KVRT_CAP_DEVICE_LENGTHS | KVRT_CAP_TENSOR_ATTEND | KVRT_CAP_PREFILL_MFMA |
           KVRT_CAP_TALKER_MASK | KVRT_CAP_PREFIX_ATTENTION | KVRT_CAP_SLOT_GENERATION | KVRT_CAP_STREAM_CONFINED |
           KVRT_CAP_ROLLBACK_POSITION;
}

const char *kvrt_strerror(int code) {
    switch (code) {
        case KVRT_OK: return "ok";
        case KVRT_EINVAL: return "invalid argument";
        case KVRT_ESTATE: return "state mismatch (length, capacity or rollback range)";
        case KVRT_EDEVICE: return "device enqueue failed; context poisoned";
        case KVRT_EPOISONED: return "context poisoned by an earlier device failure";
        case KVRT_ENOMEM: return "page pool exhausted";
        case KVRT_EFAULT: return "device-side bounds flag raised";
        default: return "unknown error";
    }
}

int kvrt_layer_storage_bytes(const kvrt_config *cfg, const kvrt_layer_spec *s, uint64_t *kv_bytes,
                             uint64_t *scale_bytes) {
    if (!cfg || !s || !kv_bytes || !scale_bytes) return KVRT_EINVAL;
    const uint64_t es = s->dtype == KVRT_INT8 ? 1 : 2;
    uint64_t rows_total;
    if (s->layout == KVRT_LAYOUT_CONTIG) rows_total = (uint64_t)cfg->n_slots * s->kv_heads * cfg->capacity;
    else if (s->layout == KVRT_LAYOUT_RING) rows_total = (uint64_t)cfg->n_slots * s->kv_heads * s->ring_rows;
    else if (s->layout == KVRT_LAYOUT_PAGED) rows_total = (uint64_t)cfg->pool_pages * s->kv_heads * cfg->block_size;
    else return KVRT_EINVAL;
    *kv_bytes = ((rows_total * s->head_dim * es + 255) / 256) * 256;
    *scale_bytes = s->dtype == KVRT_INT8 ? ((rows_total * 4 + 255) / 256) * 256 : 0;
    return KVRT_OK;
}

int kvrt_create(const kvrt_config *config, const kvrt_layer_spec *layers, kvrt_ctx **out) {
    return create_impl(config, layers, nullptr, out);
}

int kvrt_create_with_storage(const kvrt_config *config, const kvrt_layer_spec *layers,
                             const kvrt_storage *storage, kvrt_ctx **out) {
    if (!storage) return KVRT_EINVAL;
    return create_impl(config, layers, storage, out);
}

int kvrt_destroy(kvrt_ctx *c) {
    if (!c) return KVRT_EINVAL;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    else (void)hipDeviceSynchronize();
    for (Layer &L : c->layers) {
        if (!L.owned) continue;
        if (L.k) (void)hipFree(L.k);
        if (L.v) (void)hipFree(L.v);
        if (L.ks) (void)hipFree(L.ks);
        if (L.vs) (void)hipFree(L.vs);
    }
    for (Layer &L : c->layers)
        if (L.inv_freq) (void)hipFree(L.inv_freq);
    if (c->d_desc) (void)hipFree(c->d_desc);
    if (c->d_len) (void)hipFree(c->d_len);
    if (c->d_err) (void)hipFree(c->d_err);
    if (c->d_cnt) (void)hipFree(c->d_cnt);
    if (c->d_prefix) (void)hipFree(c->d_prefix);
    if (c->d_pt) (void)hipFree(c->d_pt);
    if (c->ws) (void)hipFree(c->ws);
    for (float *w : c->retired_ws) (void)hipFree(w);
    delete c;
    return KVRT_OK;
}

int kvrt_bind_stream(kvrt_ctx *c, void *stream) {
    if (!c) return KVRT_EINVAL;
    if (c->poisoned) return KVRT_EPOISONED;
    // A new context is bound to the null stream with nothing in flight.
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (c->stream == s) return KVRT_OK;
    // a switch while the bound stream may still run this context's work
    // would let two streams share its workspace and arrival counters
    if (c->dirty) return KVRT_ESTATE;
    c->stream = s;
    return KVRT_OK;
}

int kvrt_grow_slots(kvrt_ctx *c, int32_t n_slots, const kvrt_storage *storage) {
    if (!c) return KVRT_EINVAL;
    if (c->poisoned) return KVRT_EPOISONED;
    const int old_n = c->cfg.n_slots;
    if (n_slots <= old_n) return n_slots > 0 ? KVRT_OK : KVRT_EINVAL;
    if (n_slots > (1 << 20)) return KVRT_EINVAL;
    bool owns = true, slot_major = false;
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        if (c->layers[l].owner != l || c->layers[l].spec.layout == KVRT_LAYOUT_PAGED) continue;
        slot_major = true;
        owns = owns && c->layers[l].owned;
    }
    // caller-owned contexts pass the new storage; library-owned ones must not
    if (slot_major && owns == (storage != nullptr)) return KVRT_EINVAL;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(c->stream, &cs) != hipSuccess) return poison(c);
    if (cs != hipStreamCaptureStatusNone) return KVRT_ESTATE;
    kvrt_config nc = c->cfg;
    nc.n_slots = n_slots;
    // the new storage of every slot-major layer, checked before anything changes
    struct Grown { int layer; void *k, *v; uint64_t bytes, old_bytes; };
    std::vector<Grown> grown;
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        Layer &L = c->layers[l];
        if (L.owner != l || L.spec.layout == KVRT_LAYOUT_PAGED) continue;
        uint64_t kvb = 0, scb = 0;
        if (kvrt_layer_storage_bytes(&nc, &L.spec, &kvb, &scb) != KVRT_OK) return KVRT_EINVAL;
        Grown g{l, nullptr, nullptr, kvb, L.kv_bytes};
        if (storage) {
            g.k = storage[l].k;
            g.v = storage[l].v;
            if (!g.k || !g.v || ((reinterpret_cast<uintptr_t>(g.k) | reinterpret_cast<uintptr_t>(g.v)) & 15u)) {
                return KVRT_EINVAL;
            }
        }
        grown.push_back(g);
    }
    // nothing of the context may run while its buffers move
    if (hipSetDevice(c->device) != hipSuccess || hipStreamSynchronize(c->stream) != hipSuccess) return poison(c);
    c->dirty = false;
    for (Grown &g : grown) {
        if (!storage && (hipMalloc(&g.k, g.bytes) != hipSuccess || hipMalloc(&g.v, g.bytes) != hipSuccess))
            return poison(c);
        const Layer &L = c->layers[g.layer];
        // slot-major rows: the old slots are the first old_bytes, the new ones start zeroed
        if (hipMemcpyAsync(g.k, L.k, g.old_bytes, hipMemcpyDeviceToDevice, c->stream) != hipSuccess ||
            hipMemcpyAsync(g.v, L.v, g.old_bytes, hipMemcpyDeviceToDevice, c->stream) != hipSuccess)
            return poison(c);
        const uint64_t tail = g.bytes - g.old_bytes;
        if (launch_zero(static_cast<uint8_t *>(g.k) + g.old_bytes, tail, c->stream) != hipSuccess ||
            launch_zero(static_cast<uint8_t *>(g.v) + g.old_bytes, tail, c->stream) != hipSuccess)
            return poison(c);
    }
    // lengths [slot, layer], page table [slot, page] and masks [slot]: slot-major, new rows appended
    int32_t *d_len = nullptr, *d_pt = nullptr;
    PrefixMask *d_prefix = nullptr;
    const size_t len_old = c->len.size() * 4, len_new = (size_t)n_slots * c->cfg.n_layers * 4;
    const size_t len_alloc = ((len_new + 15) / 16) * 16;
    if (hipMalloc((void **)&d_len, len_alloc) != hipSuccess || launch_zero(d_len, len_alloc, c->stream) != hipSuccess ||
        hipMemcpyAsync(d_len, c->d_len, len_old, hipMemcpyDeviceToDevice, c->stream) != hipSuccess)
        return poison(c);
    if (hipMalloc((void **)&d_prefix, (size_t)n_slots * sizeof(PrefixMask)) != hipSuccess ||
        launch_zero(d_prefix, (size_t)n_slots * sizeof(PrefixMask), c->stream) != hipSuccess ||
        hipMemcpyAsync(d_prefix, c->d_prefix, (size_t)old_n * sizeof(PrefixMask), hipMemcpyDeviceToDevice,
                       c->stream) != hipSuccess)
        return poison(c);
    if (c->paged) {
        std::vector<int32_t> pt = c->pt;
        pt.resize((size_t)n_slots * c->pt_stride, -1);
        const size_t pt_bytes = ((pt.size() * 4 + 15) / 16) * 16;
        if (hipMalloc((void **)&d_pt, pt_bytes) != hipSuccess ||
            hipMemcpy(d_pt, pt.data(), pt.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return poison(c);
        c->pt = std::move(pt);
        c->first_live.resize(n_slots, 0);
    }
    if (hipStreamSynchronize(c->stream) != hipSuccess) return poison(c);
    for (Grown &g : grown) {
        Layer &L = c->layers[g.layer];
        if (L.owned) {
            (void)hipFree(L.k);
            (void)hipFree(L.v);
        }
        L.k = g.k;
        L.v = g.v;
        L.kv_bytes = g.bytes;
    }
    (void)hipFree(c->d_len);
    (void)hipFree(c->d_prefix);
    c->d_len = d_len;
    c->d_prefix = d_prefix;
    if (c->paged) {
        (void)hipFree(c->d_pt);
        c->d_pt = d_pt;
    }
    c->len.resize((size_t)n_slots * c->cfg.n_layers, 0);
    c->ring_lo.resize((size_t)n_slots * c->cfg.n_layers, 0);
    c->slot.resize(n_slots, SlotState{});
    for (int i = old_n; i < n_slots; ++i) renew_generation(c, i);
    c->cfg.n_slots = n_slots;
    if (upload_desc(c) != KVRT_OK) return poison(c);
    if (ensure_workspace(c, workspace_bound(c)) != KVRT_OK) return poison(c);
    return hipDeviceSynchronize() == hipSuccess ? KVRT_OK : poison(c);
}

int kvrt_layer_storage(kvrt_ctx *c, int32_t layer, kvrt_storage *out) {
    if (!c || !out || !valid_layer(c, layer)) return KVRT_EINVAL;
    const Layer &L = c->layers[c->layers[layer].owner];
    out->k = L.k;
    out->v = L.v;
    out->k_scale = L.ks;
    out->v_scale = L.vs;
    return KVRT_OK;
}

int kvrt_import_async(kvrt_ctx *c, int32_t slot, int32_t layer, const kvrt_tensor *k, const kvrt_tensor *v,
                      int32_t first_pos) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_slot(c, slot) || !valid_layer(c, layer)) return KVRT_EINVAL;
    if (c->layers[layer].owner != layer) return KVRT_EINVAL;  // import the source layer instead
    const kvrt_layer_spec &s = c->layers[layer].spec;
    if (!tensor_ok_or_empty(k, KVRT_BF16, 4) || !tensor_ok_or_empty(v, KVRT_BF16, 4)) return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (k->dims[i] != v->dims[i] || (k->dims[2] > 0 && k->strides[i] != v->strides[i])) return KVRT_EINVAL;
    const int64_t S = k->dims[2];
    if (k->dims[0] != 1 || k->dims[1] != s.kv_heads || k->dims[3] != s.head_dim) return KVRT_EINVAL;
    if (S < 0 || S > c->cfg.capacity || first_pos < 0 || first_pos > S) return KVRT_EINVAL;
    // an import starts a session: never over one that is live (rows on this
    // layer, or a prefix mask), import_cache_async's `primed` refusal; the
    // host must vouch for the lengths it checks
    if (c->len_at(slot, layer) != 0 || c->slot[slot].prefix_len != 0 || c->lens_stale) return KVRT_ESTATE;
    int keep_from = first_pos;
    std::vector<int32_t> pidx, pval;
    if (s.layout == KVRT_LAYOUT_RING) {
        keep_from = std::max<int64_t>(keep_from, S - s.ring_rows);
    } else if (s.layout == KVRT_LAYOUT_PAGED) {
        keep_from = (first_pos / c->cfg.block_size) * c->cfg.block_size;
        rc = map_pages(c, slot, keep_from, (int)S, pidx, pval);
        if (rc) return rc;
        rc = enqueue_pages(c, pidx, pval);
        if (rc) return rc;
        c->first_live[slot] = std::max(c->first_live[slot], keep_from / c->cfg.block_size);
    }
    AppendArgs a{};
    a.kv = make_view(c, layer);
    a.len = make_len(c, layer);
    a.k_src = static_cast<const uint16_t *>(k->data);
    a.v_src = static_cast<const uint16_t *>(v->data);
    a.src_item_stride = 0;
    a.src_head_stride = k->strides[1];
    a.src_row_stride = k->strides[2];
    a.n_items = 1;
    a.rows = (int)S;
    a.import_mode = 1;
    a.base_pos = 0;
    a.keep_from = keep_from;
    a.err = c->d_err;
    a.slots[0] = slot;
    if (S > 0) {
        const int64_t chunks = (int64_t)s.kv_heads * S * (s.head_dim / 8);
        int gx = (int)std::min<int64_t>(4096, (chunks + 255) / 256);
        c->counters.launches++;
        if (launch_append(a, s.head_dim, s.dtype, std::max(1, gx), enq(c)) != hipSuccess) return poison(c);
    } else {
        std::vector<int32_t> idx{(int32_t)((size_t)slot * c->cfg.n_layers + layer)};
        c->len_ref(slot, layer) = 0;
        rc = set_device_lens(c, idx);
        if (rc) return rc;
    }
    c->len_ref(slot, layer) = (int)S;
    c->ring_set(slot, layer, s.layout == KVRT_LAYOUT_RING ? keep_from : 0);  // rows below keep_from are not written
    c->counters.appended_rows += (uint64_t)S * s.kv_heads;
    c->counters.appended_bytes += (uint64_t)S * s.kv_heads * s.head_dim * 2 * (s.dtype == KVRT_INT8 ? 1 : 2);
    // new contents: holders of the slot's previous generation are stale
    renew_generation(c, slot);
    return KVRT_OK;
}

int kvrt_append_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const kvrt_tensor *k,
                      const kvrt_tensor *v) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots)) return KVRT_EINVAL;
    return append_impl(c, layer, n, slots, k, v);
}

int kvrt_write_positions_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots,
                               const int32_t *positions, const kvrt_tensor *k, const kvrt_tensor *v) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots) || !positions) return KVRT_EINVAL;
    if (c->layers[layer].owner != layer) return KVRT_EINVAL;  // shared layers own no rows
    const kvrt_layer_spec &s = c->layers[layer].spec;
    if (s.layout != KVRT_LAYOUT_CONTIG || s.dtype != KVRT_BF16) return KVRT_EINVAL;
    const int D = s.head_dim, hkv = s.kv_heads;
    if (!tensor_ok(k, KVRT_BF16, 4) || !tensor_ok(v, KVRT_BF16, 4)) return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (k->dims[i] != v->dims[i] || k->strides[i] != v->strides[i]) return KVRT_EINVAL;
    const int64_t qn = k->dims[2];
    if (k->dims[0] != n || k->dims[1] != hkv || k->dims[3] != D || (int64_t)n * qn > kMaxPositions)
        return KVRT_EINVAL;
    if (qn == 0) return KVRT_OK;  // an empty write leaves every length unchanged
    AppendArgs a{};
    for (int i = 0; i < n; ++i) {
        int end = 0;
        for (int r = 0; r < qn; ++r) {
            const int p = positions[i * qn + r];
            if (p < 0 || p >= c->cfg.capacity) return KVRT_ESTATE;
            for (int r2 = 0; r2 < r; ++r2)
                if (positions[i * qn + r2] == p) return KVRT_EINVAL;  // two rows, one position
            end = std::max(end, p + 1);
            a.pos[i * qn + r] = p;
        }
        a.pos_end[i] = end;
        a.slots[i] = slots[i];
    }
    a.kv = make_view(c, layer);
    a.len = make_len(c, layer);
    a.k_src = static_cast<const uint16_t *>(k->data);
    a.v_src = static_cast<const uint16_t *>(v->data);
    a.src_item_stride = k->strides[0];
    a.src_head_stride = k->strides[1];
    a.src_row_stride = k->strides[2];
    a.n_items = n;
    a.rows = (int)qn;
    a.import_mode = 2;
    a.err = c->d_err;
    c->counters.launches++;
    if (launch_append(a, D, s.dtype, 1, enq(c)) != hipSuccess) return poison(c);
    for (int i = 0; i < n; ++i) {
        int &L = c->len_ref(slots[i], layer);
        L = std::max(L, a.pos_end[i]);
        c->counters.appended_rows += (uint64_t)qn * hkv;
        c->counters.appended_bytes += (uint64_t)qn * hkv * D * 2 * 2;
    }
    return KVRT_OK;
}

int kvrt_reset_slot_async(kvrt_ctx *c, int32_t slot) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_slot(c, slot)) return KVRT_EINVAL;
    std::vector<int32_t> idx;
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        if (c->layers[l].owner != l) continue;
        const kvrt_layer_spec &s = c->layers[l].spec;
        if (s.layout != KVRT_LAYOUT_PAGED) {
            const KVView vw = make_view(c, l);
            const uint64_t bytes = (uint64_t)vw.slot_stride * 2;
            for (void *base : {vw.k, vw.v}) {
                c->counters.launches++;
                if (launch_zero(static_cast<uint8_t *>(base) + (uint64_t)slot * bytes, bytes, enq(c)) != hipSuccess)
                    return poison(c);
            }
        }
        c->len_ref(slot, l) = 0;
        c->ring_set(slot, l, 0);
        idx.push_back((int32_t)((size_t)slot * c->cfg.n_layers + l));
    }
    if (c->paged) {
        for (int p = 0; p < c->pt_stride; ++p) {
            int32_t &e = c->pt[(size_t)slot * c->pt_stride + p];
            if (e >= 0) {
                c->free_pages.push_back(e);
                e = -1;
                c->counters.pages_in_use--;
            }
        }
        c->first_live[slot] = 0;
    }
    rc = set_device_lens(c, idx);
    if (rc != KVRT_OK) return rc;
    rc = set_prefix_len_device(c, slot, 0);
    if (rc != KVRT_OK) return rc;
    renew_generation(c, slot);
    return KVRT_OK;
}

int kvrt_set_prefix_attention_async(kvrt_ctx *c, int32_t slot, const kvrt_tensor *mask) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_slot(c, slot)) return KVRT_EINVAL;
    PrefixPackArgs a{};
    if (mask != nullptr) {
        rc = prefix_tensor(mask, 1, a);
        if (rc != KVRT_OK) return rc;
    }
    if (a.plen == 0) return set_prefix_len_device(c, slot, 0);
    // the masked positions must be in the slot already (the mask comes with
    // an imported prefix), so that the rewind floor holds from the start
    for (int l = 0; l < c->cfg.n_layers; ++l)
        if (c->layers[l].owner == l && c->len_at(slot, l) < a.plen) return KVRT_ESTATE;
    a.dst = c->d_prefix;
    a.index[0] = slot;
    c->counters.launches++;
    if (launch_prefix_pack(a, enq(c)) != hipSuccess) return poison(c);
    c->slot[slot].prefix_len = a.plen;
    return KVRT_OK;
}

int kvrt_slot_info_get(kvrt_ctx *c, int32_t slot, kvrt_slot_info *out) {
    if (!c || !out || !valid_slot(c, slot)) return KVRT_EINVAL;
    kvrt_slot_info r{};
    r.generation = c->slot[slot].generation;
    r.prefix_len = c->slot[slot].prefix_len;
    r.min_len = INT32_MAX;
    r.max_len = 0;
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        if (c->layers[l].owner != l) continue;
        r.min_len = std::min(r.min_len, c->len_at(slot, l));
        r.max_len = std::max(r.max_len, c->len_at(slot, l));
    }
    if (r.min_len == INT32_MAX) r.min_len = 0;
    *out = r;
    return KVRT_OK;
}

// Gather, and with k / v the append of their rows fused into the same launch
// (bf16 CONTIG / RING layers that own their rows, at most max_q rows; the
// caller has validated the context, layer and slots).
static int gather_impl(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const int32_t *start_pos,
                       const kvrt_tensor *out_k, const kvrt_tensor *out_v, const kvrt_tensor *mask,
                       const kvrt_tensor *k, const kvrt_tensor *v) {
    const kvrt_layer_spec &s = c->layers[layer].spec;
    int qn = 0;
    if (k) {
        const int D = s.head_dim, hkv = s.kv_heads;
        if (!tensor_ok(k, KVRT_BF16, 4) || !tensor_ok(v, KVRT_BF16, 4) || !is_contiguous(k) || !is_contiguous(v))
            return KVRT_EINVAL;
        for (int i = 0; i < 4; ++i)
            if (k->dims[i] != v->dims[i]) return KVRT_EINVAL;
        if (k->dims[0] != n || k->dims[1] != hkv || k->dims[3] != D || k->dims[2] < 1 || k->dims[2] > c->cfg.max_q)
            return KVRT_EINVAL;
        qn = (int)k->dims[2];
        for (int i = 0; i < n; ++i)
            if ((int64_t)c->len_at(slots[i], layer) + qn > c->cfg.capacity) return KVRT_ESTATE;
    }
    const int out_dtype = s.dtype == KVRT_INT8 ? KVRT_FP32 : KVRT_BF16;
    if (!tensor_ok(out_k, out_dtype, 4) || !tensor_ok(out_v, out_dtype, 4)) return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (out_k->dims[i] != out_v->dims[i] || out_k->strides[i] != out_v->strides[i]) return KVRT_EINVAL;
    const int64_t lmax = out_k->dims[2];
    if (out_k->dims[0] != n || out_k->dims[1] != s.kv_heads || out_k->dims[3] != s.head_dim || lmax <= 0 ||
        lmax > (1 << 30))
        return KVRT_EINVAL;
    if (mask) {
        if (!mask->data || mask->ndim != 2 || mask->dims[0] != n || mask->dims[1] != lmax || mask->strides[1] != 1)
            return KVRT_EINVAL;
        if (mask->dtype != KVRT_BOOL && mask->dtype != KVRT_FP32 && mask->dtype != KVRT_BF16) return KVRT_EINVAL;
    }
    GatherArgs a{};
    for (int i = 0; i < n; ++i) {
        const int L = c->len_at(slots[i], layer) + qn;
        int st;
        if (start_pos) st = start_pos[i];
        else if (s.layout == KVRT_LAYOUT_RING) st = std::max(0, L - (s.window - 1));
        else if (s.layout == KVRT_LAYOUT_PAGED) st = std::min(L, c->first_live[slots[i]] * c->cfg.block_size);
        else st = 0;
        if (st < 0 || st > L || L - st > lmax) return KVRT_EINVAL;
        if (s.layout == KVRT_LAYOUT_RING && st < std::max(L - s.ring_rows, c->ring_floor(slots[i], layer)))
            return KVRT_ESTATE;
        if (s.layout == KVRT_LAYOUT_PAGED) {
            for (int p = st / c->cfg.block_size; p * c->cfg.block_size < L; ++p)
                if (c->pt[(size_t)slots[i] * c->pt_stride + p] < 0) return KVRT_ESTATE;
        }
        a.start[i] = st;
        a.slots[i] = slots[i];
    }
    // RING without start_pos: the kernel derives max(0, L - (W - 1)) from
    // the device length, so a captured call replays with the window moving
    // along (the host value above only validates this call); CONTIG starts
    // at 0 either way; PAGED starts at the host's first live page
    a.has_start = start_pos != nullptr || s.layout == KVRT_LAYOUT_PAGED;
    a.kv = make_view(c, layer);
    a.len = make_len(c, layer);
    a.out_k = out_k->data;
    a.out_v = out_v->data;
    a.out_item_stride = out_k->strides[0];
    a.out_head_stride = out_k->strides[1];
    a.out_row_stride = out_k->strides[2];
    a.mask = mask ? mask->data : nullptr;
    a.mask_item_stride = mask ? mask->strides[0] : 0;
    a.mask_dtype = mask ? mask->dtype : KVRT_BOOL;
    a.out_fp32 = out_dtype == KVRT_FP32;
    a.n_items = n;
    a.lmax = (int)lmax;
    a.window = s.window;
    a.err = c->d_err;
    if (k) {
        a.k_new = static_cast<const uint16_t *>(k->data);
        a.v_new = static_cast<const uint16_t *>(v->data);
        a.cnt = c->d_cnt;
        a.qn = qn;
    }
    c->counters.launches++;
    if (launch_gather(a, s.head_dim, s.dtype, enq(c)) != hipSuccess) return poison(c);
    c->counters.gathered_bytes += (uint64_t)n * s.kv_heads * lmax * s.head_dim * 2 * elem_size(out_dtype);
    for (int i = 0; k && i < n; ++i) {
        c->len_ref(slots[i], layer) += qn;
        c->ring_advance(slots[i], layer);
        c->counters.appended_rows += (uint64_t)qn * s.kv_heads;
        c->counters.appended_bytes += (uint64_t)qn * s.kv_heads * s.head_dim * 2 * 2;
    }
    return KVRT_OK;
}

int kvrt_gather_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const int32_t *start_pos,
                      const kvrt_tensor *out_k, const kvrt_tensor *out_v, const kvrt_tensor *mask) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots)) return KVRT_EINVAL;
    return gather_impl(c, layer, n, slots, start_pos, out_k, out_v, mask, nullptr, nullptr);
}

int kvrt_append_gather_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const kvrt_tensor *k,
                             const kvrt_tensor *v, const int32_t *start_pos, const kvrt_tensor *out_k,
                             const kvrt_tensor *out_v, const kvrt_tensor *mask) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots) || !k || !v) return KVRT_EINVAL;
    const kvrt_layer_spec &s = c->layers[layer].spec;
    const bool fusable = c->layers[layer].owner == layer && s.dtype == KVRT_BF16 && s.layout != KVRT_LAYOUT_PAGED &&
                         k->ndim == 4 && k->dims[2] >= 1 && k->dims[2] <= c->cfg.max_q && is_contiguous(k) &&
                         is_contiguous(v);
    if (fusable) return gather_impl(c, layer, n, slots, start_pos, out_k, out_v, mask, k, v);
    // shared layers (no rows of their own), PAGED and int8 layers, longer
    // appends: the append launch, then the gather
    rc = append_impl(c, layer, n, slots, k, v);
    if (rc != KVRT_OK) return rc;
    return gather_impl(c, layer, n, slots, start_pos, out_k, out_v, mask, nullptr, nullptr);
}

int kvrt_truncate(kvrt_ctx *c, int32_t slot, int32_t layer, int32_t new_len, uint64_t expected_generation,
                  int32_t expected_len) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_slot(c, slot) || layer < -1 || layer >= c->cfg.n_layers || new_len < 0 || expected_len < -1)
        return KVRT_EINVAL;
    // identity and the rewind floor: the prefix-attention mask's positions
    // stay; lengths the host cannot vouch for (captured work since the last
    // read-back) refuse the rollback
    if (!generation_ok(c, slot, expected_generation) || new_len < c->slot[slot].prefix_len || c->lens_stale)
        return KVRT_ESTATE;
    std::vector<int> targets;
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        if (layer >= 0 && l != layer) continue;
        if (c->layers[l].owner != l) continue;
        targets.push_back(l);
    }
    if (layer >= 0 && targets.empty()) targets.push_back(c->layers[layer].owner);
    for (int l : targets) {
        const kvrt_layer_spec &s = c->layers[l].spec;
        const int L = c->len_at(slot, l);
        // the caller's position must be the slot's (rewind_session_async's
        // current_position == valid_kv_len)
        if (new_len > L || (expected_len >= 0 && L != expected_len)) return KVRT_ESTATE;
        // The keys the next query (position new_len) sees must still be
        // stored: in the ring (RING), on live pages (PAGED with a window;
        // without one, no rollback into released pages). A rollback to 0
        // keeps no rows (a release) and is always possible.
        if (new_len == 0 || new_len == L) continue;
        const int need = s.window > 0 ? std::max(0, new_len - s.window + 1) : new_len;
        if (s.layout == KVRT_LAYOUT_RING && need < c->ring_floor(slot, l)) return KVRT_ESTATE;
        if (s.layout == KVRT_LAYOUT_PAGED && need < c->first_live[slot] * c->cfg.block_size) return KVRT_ESTATE;
    }
    std::vector<int32_t> idx, before;
    for (int l : targets) {
        int &L = c->len_ref(slot, l);
        if (L == new_len) continue;
        c->counters.truncated_rows += (uint64_t)(L - new_len);
        before.push_back(L);
        L = new_len;
        if (new_len == 0) c->ring_set(slot, l, 0);
        idx.push_back((int32_t)((size_t)slot * c->cfg.n_layers + l));
    }
    if (c->paged) {
        // Release pages wholly beyond the longest remaining paged layer.
        int keep = 0;
        for (int l = 0; l < c->cfg.n_layers; ++l)
            if (c->layers[l].owner == l && c->layers[l].spec.layout == KVRT_LAYOUT_PAGED)
                keep = std::max(keep, c->len_at(slot, l));
        const int bs = c->cfg.block_size;
        for (int p = (keep + bs - 1) / bs; p < c->pt_stride; ++p) {
            int32_t &e = c->pt[(size_t)slot * c->pt_stride + p];
            if (e >= 0) {
                c->free_pages.push_back(e);
                e = -1;
                c->counters.pages_in_use--;
            }
        }
        if (keep == 0) c->first_live[slot] = 0;
    }
    c->counters.truncations++;
    return set_device_lens(c, idx, &before);
}

int kvrt_reserve_async(kvrt_ctx *c, int32_t slot, int32_t positions) {
    int rc = begin(c);
    if (rc) return rc;
    if (!c->paged || !valid_slot(c, slot) || positions < 0) return KVRT_EINVAL;
    if (c->lens_stale) return KVRT_ESTATE;  // the host must vouch for the length it maps from
    int L = 0;  // pages are per slot: from the longest PAGED layer on
    for (int l = 0; l < c->cfg.n_layers; ++l)
        if (c->layers[l].owner == l && c->layers[l].spec.layout == KVRT_LAYOUT_PAGED) L = std::max(L, c->len_at(slot, l));
    if ((int64_t)L + positions > c->cfg.capacity) return KVRT_ESTATE;
    std::vector<int32_t> idx, val;
    rc = map_pages(c, slot, L, L + positions, idx, val);
    if (rc != KVRT_OK) return rc;
    return enqueue_pages(c, idx, val);
}

int kvrt_evict(kvrt_ctx *c, int32_t slot, int32_t keep_from) {
    int rc = begin(c);
    if (rc) return rc;
    if (!c->paged || !valid_slot(c, slot) || keep_from < 0) return KVRT_EINVAL;
    const int bs = c->cfg.block_size;
    const int last = keep_from / bs;  // pages [0, last) are wholly below keep_from
    for (int p = c->first_live[slot]; p < last && p < c->pt_stride; ++p) {
        int32_t &e = c->pt[(size_t)slot * c->pt_stride + p];
        if (e >= 0) {
            c->free_pages.push_back(e);
            e = -1;
            c->counters.pages_in_use--;
            c->counters.pages_evicted++;
        }
    }
    c->first_live[slot] = std::max(c->first_live[slot], std::min(last, c->pt_stride));
    return KVRT_OK;
}

namespace {

// Positions [lo, n) of (slot, layer) that a copy of the first n tokens
// carries: CONTIG all of them, RING those still in the ring, PAGED those on
// live pages. KVRT_ESTATE when a key the next query (position n) can see is
// not resident.
int copy_range(const kvrt_ctx *c, int slot, int l, int n, int &lo) {
    const kvrt_layer_spec &s = c->layers[l].spec;
    const int L = c->len_at(slot, l);
    if (n > L) return KVRT_ESTATE;
    lo = 0;
    if (n == 0) return KVRT_OK;  // nothing to carry
    const int need = s.window > 0 ? std::max(0, n - s.window + 1) : 0;
    if (s.layout == KVRT_LAYOUT_RING) lo = std::max({0, n - s.ring_rows, L - s.ring_rows, c->ring_floor(slot, l)});
    else if (s.layout == KVRT_LAYOUT_PAGED) lo = std::min(n, c->first_live[slot] * c->cfg.block_size);
    return lo > need ? KVRT_ESTATE : KVRT_OK;
}

bool same_topology(const kvrt_ctx *a, const kvrt_ctx *b) {
    if (a->cfg.n_layers != b->cfg.n_layers || a->device != b->device) return false;
    if (a->paged != b->paged || (a->paged && a->cfg.block_size != b->cfg.block_size)) return false;
    for (int l = 0; l < a->cfg.n_layers; ++l) {
        const kvrt_layer_spec &x = a->layers[l].spec, &y = b->layers[l].spec;
        if (x.layout != y.layout || x.dtype != y.dtype || x.kv_heads != y.kv_heads || x.head_dim != y.head_dim ||
            x.window != y.window || x.ring_rows != y.ring_rows || a->layers[l].owner != b->layers[l].owner)
            return false;
    }
    return true;
}

// Copy the first n tokens of every owned layer of (src, src_slot) into
// (dst, dst_slot), on dst's stream; dst lengths become n.
int copy_slot_impl(kvrt_ctx *dst, int dst_slot, kvrt_ctx *src, int src_slot, int n, uint64_t src_generation) {
    if (!generation_ok(src, src_slot, src_generation)) return KVRT_ESTATE;
    const int src_plen = src->slot[src_slot].prefix_len;
    if (n < src_plen) return KVRT_ESTATE;  // the copy would end inside the masked prefix
    const int nl = src->cfg.n_layers;
    std::vector<int> lo(nl, 0);
    int page_lo = n;
    for (int l = 0; l < nl; ++l) {
        if (src->layers[l].owner != l) continue;
        const kvrt_layer_spec &s = src->layers[l].spec;
        if (s.layout == KVRT_LAYOUT_CONTIG && n > dst->cfg.capacity) return KVRT_ESTATE;
        const int rc = copy_range(src, src_slot, l, n, lo[l]);
        if (rc != KVRT_OK) return rc;
        if (s.layout == KVRT_LAYOUT_PAGED) page_lo = std::min(page_lo, lo[l]);
    }
    // destination pages: release what the slot holds (host bookkeeping only:
    // the device table is read only inside mapped, live ranges), then map the
    // copied range; only the new mappings are enqueued, each index once
    std::vector<int32_t> pidx, pval;
    if (dst->paged) {
        const int bs = dst->cfg.block_size;
        const int need = n > 0 ? (n - 1) / bs - page_lo / bs + 1 : 0;
        if ((n - 1) / bs >= dst->pt_stride) return KVRT_ESTATE;
        int held = 0;
        for (int p = 0; p < dst->pt_stride; ++p) held += dst->pt[(size_t)dst_slot * dst->pt_stride + p] >= 0;
        if (need > (int)dst->free_pages.size() + held) return KVRT_ENOMEM;  // nothing changed
        for (int p = 0; p < dst->pt_stride; ++p) {
            int32_t &e = dst->pt[(size_t)dst_slot * dst->pt_stride + p];
            if (e >= 0) {
                dst->free_pages.push_back(e);
                e = -1;
                dst->counters.pages_in_use--;
            }
        }
        const int from = (page_lo / bs) * bs;
        if (map_pages(dst, dst_slot, from, n, pidx, pval) != KVRT_OK) return poison(dst);  // counted above
        dst->first_live[dst_slot] = from / bs;
    }
    int rc = enqueue_pages(dst, pidx, pval);
    if (rc != KVRT_OK) return rc;
    SlotMoveArgs a{};
    a.src = src->d_desc;
    a.dst = dst->d_desc;
    a.err = dst->d_err;
    a.src_slot = src_slot;
    a.dst_slot = dst_slot;
    int64_t max_units = 0;
    uint64_t bytes = 0;
    auto flush = [&]() -> int {
        if (a.n_entries == 0) return KVRT_OK;
        dst->counters.launches++;
        if (launch_slot_copy(a, max_units, enq(dst)) != hipSuccess) return poison(dst);
        a.n_entries = 0;
        max_units = 0;
        return KVRT_OK;
    };
    std::vector<int32_t> idx;
    for (int l = 0; l < nl; ++l) {
        if (src->layers[l].owner != l) continue;
        const kvrt_layer_spec &s = src->layers[l].spec;
        const int rows = n - lo[l];
        if (rows > 0) {
            const int e = a.n_entries++;
            a.layer[e] = l;
            a.src_pos0[e] = a.dst_pos0[e] = lo[l];
            a.rows[e] = rows;
            const int eb = s.dtype == KVRT_INT8 ? 1 : 2;
            max_units = std::max<int64_t>(max_units, (int64_t)s.kv_heads * rows * (s.head_dim * eb / 16));
            bytes += (uint64_t)rows * s.kv_heads * (s.head_dim * eb + (eb == 1 ? 8 : 0)) * 2;
            if (a.n_entries == kMaxMoveLayers && (rc = flush()) != KVRT_OK) return rc;
        }
        dst->len_ref(dst_slot, l) = n;
        dst->ring_set(dst_slot, l, s.layout == KVRT_LAYOUT_RING ? lo[l] : 0);
        idx.push_back((int32_t)((size_t)dst_slot * nl + l));
    }
    if ((rc = flush()) != KVRT_OK) return rc;
    dst->counters.gathered_bytes += bytes;
    rc = set_device_lens(dst, idx);
    if (rc != KVRT_OK) return rc;
    // the prefix-attention mask travels with the rows (a 128-byte record)
    CopyRowsArgs m{};
    m.src = reinterpret_cast<const uint8_t *>(src->d_prefix + src_slot);
    m.dst = reinterpret_cast<uint8_t *>(dst->d_prefix + dst_slot);
    m.d0 = m.d1 = m.rows = 1;
    m.row_bytes = sizeof(PrefixMask);
    dst->counters.launches++;
    if (launch_copy_rows(m, enq(dst)) != hipSuccess) return poison(dst);
    dst->slot[dst_slot].prefix_len = src_plen;
    renew_generation(dst, dst_slot);
    return KVRT_OK;
}

}  // namespace

int kvrt_copy_prefix_async(kvrt_ctx *c, int32_t src_slot, int32_t dst_slot, int32_t n_tokens,
                           uint64_t src_generation) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_slot(c, src_slot) || !valid_slot(c, dst_slot) || src_slot == dst_slot || n_tokens < 0)
        return KVRT_EINVAL;
    return copy_slot_impl(c, dst_slot, c, src_slot, n_tokens, src_generation);
}

int kvrt_copy_session_async(kvrt_ctx *dst, int32_t dst_slot, kvrt_ctx *src, int32_t src_slot, int32_t n_tokens,
                            uint64_t src_generation) {
    if (!dst || !src || dst == src) return KVRT_EINVAL;
    if (src->poisoned) return KVRT_EPOISONED;
    int rc = begin(dst);
    if (rc) return rc;
    if (!valid_slot(dst, dst_slot) || !valid_slot(src, src_slot) || n_tokens < 0) return KVRT_EINVAL;
    if (!same_topology(dst, src)) return KVRT_EINVAL;
    return copy_slot_impl(dst, dst_slot, src, src_slot, n_tokens, src_generation);
}

int kvrt_set_layer_rope(kvrt_ctx *c, int32_t layer, const float *inv_freq, int32_t n_freq, float scaling) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || c->layers[layer].owner != layer) return KVRT_EINVAL;
    Layer &L = c->layers[layer];
    if (L.spec.dtype != KVRT_BF16 || !std::isfinite(scaling)) return KVRT_EINVAL;
    if (inv_freq == nullptr) {
        if (n_freq != 0) return KVRT_EINVAL;
    } else {
        if (n_freq != L.spec.head_dim / 2) return KVRT_EINVAL;
        for (int i = 0; i < n_freq; ++i)
            if (!std::isfinite(inv_freq[i])) return KVRT_EINVAL;
    }
    // pending work may read the current table
    if (hipStreamSynchronize(c->stream) != hipSuccess) return poison(c);
    c->dirty = false;
    if (inv_freq == nullptr) {
        if (L.inv_freq) (void)hipFree(L.inv_freq);
        L.inv_freq = nullptr;
    } else {
        if (!L.inv_freq && hipMalloc((void **)&L.inv_freq, (size_t)n_freq * sizeof(float)) != hipSuccess)
            return poison(c);
        if (hipMemcpy(L.inv_freq, inv_freq, (size_t)n_freq * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            return poison(c);
    }
    L.rope_scaling = scaling;
    return upload_desc(c) == KVRT_OK ? KVRT_OK : poison(c);
}

int kvrt_rollover_async(kvrt_ctx *c, int32_t slot, int32_t prefix_len, int32_t retained_rows,
                        uint64_t expected_generation) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_slot(c, slot) || prefix_len <= 0 || retained_rows <= 0 || retained_rows > KVRT_MAX_ROLLOVER_ROWS)
        return KVRT_EINVAL;
    if (!generation_ok(c, slot, expected_generation) || prefix_len < c->slot[slot].prefix_len) return KVRT_ESTATE;
    int L = -1, max_heads = 0;
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        if (c->layers[l].owner != l) continue;
        const kvrt_layer_spec &s = c->layers[l].spec;
        if (s.layout == KVRT_LAYOUT_RING || s.dtype != KVRT_BF16) return KVRT_EINVAL;
        const int Ll = c->len_at(slot, l);
        if (L >= 0 && Ll != L) return KVRT_ESTATE;
        L = Ll;
        max_heads = std::max(max_heads, s.kv_heads);
    }
    if (L < 0) return KVRT_EINVAL;
    if ((int64_t)L <= (int64_t)prefix_len + retained_rows) return KVRT_ESTATE;
    if (c->paged && c->first_live[slot] > 0) return KVRT_ESTATE;  // the prefix pages are gone
    SlotMoveArgs a{};
    a.src = a.dst = c->d_desc;
    a.err = c->d_err;
    a.src_slot = a.dst_slot = slot;
    a.rope_delta = prefix_len - (L - retained_rows);
    std::vector<int32_t> idx;
    uint64_t bytes = 0;
    for (int l = 0; l < c->cfg.n_layers; ++l) {
        if (c->layers[l].owner != l) continue;
        const kvrt_layer_spec &s = c->layers[l].spec;
        const int e = a.n_entries++;
        a.layer[e] = l;
        a.src_pos0[e] = L - retained_rows;
        a.dst_pos0[e] = prefix_len;
        a.rows[e] = retained_rows;
        bytes += (uint64_t)retained_rows * s.kv_heads * s.head_dim * 2 * 2;
        if (a.n_entries == kMaxMoveLayers) {
            c->counters.launches++;
            if (launch_slot_rebase(a, max_heads, enq(c)) != hipSuccess) return poison(c);
            a.n_entries = 0;
        }
        c->len_ref(slot, l) = prefix_len + retained_rows;
        idx.push_back((int32_t)((size_t)slot * c->cfg.n_layers + l));
    }
    if (a.n_entries) {
        c->counters.launches++;
        if (launch_slot_rebase(a, max_heads, enq(c)) != hipSuccess) return poison(c);
    }
    c->counters.truncations++;
    c->counters.truncated_rows += (uint64_t)(L - prefix_len - retained_rows) * idx.size();
    c->counters.gathered_bytes += bytes;
    return set_device_lens(c, idx);
}

int kvrt_attend_decode_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const kvrt_tensor *q,
                             const kvrt_tensor *out, float scale) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots)) return KVRT_EINVAL;
    return decode_impl(c, layer, n, slots, q, nullptr, nullptr, out, scale);
}

int kvrt_attend_talker_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const kvrt_tensor *q,
                             const kvrt_tensor *out, float scale, const kvrt_talker_mask *masks) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots) || !masks) return KVRT_EINVAL;
    return decode_impl(c, layer, n, slots, q, nullptr, nullptr, out, scale, masks);
}

int kvrt_append_attend_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const kvrt_tensor *q,
                             const kvrt_tensor *k, const kvrt_tensor *v, const kvrt_tensor *out, float scale) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots) || !k || !v) return KVRT_EINVAL;
    if (c->layers[layer].owner != layer) return KVRT_EINVAL;  // shared layers append nothing
    const kvrt_layer_spec &ls = c->layers[layer].spec;
    if (ls.dtype == KVRT_INT8 && c->cfg.decode_kernel == KVRT_DECODE_MFMA) {
        // the register-staged MFMA decode reads int8 rows only: the append
        // kernel quantises them first (the int8 ring kernel quantises them
        // in its own launch)
        int64_t rows = 0;
        if (tensor_ok(q, KVRT_BF16, 4) && q->dims[1] % ls.kv_heads == 0) rows = q->dims[1] / ls.kv_heads * q->dims[2];
        if (!(rows > 0 && rows <= 16 && i8_mfma_dma(ls.head_dim, rows_tile((int)rows)))) {
            rc = append_impl(c, layer, n, slots, k, v);
            if (rc) return rc;
            return decode_impl(c, layer, n, slots, q, nullptr, nullptr, out, scale);
        }
    }
    // one launch: the decode stores the new rows (int8: quantised in-kernel)
    return decode_impl(c, layer, n, slots, q, k, v, out, scale);
}

int kvrt_attend_prefill_async(kvrt_ctx *c, int32_t layer, int32_t n, const int32_t *slots, const kvrt_tensor *q,
                              const kvrt_tensor *out, float scale) {
    int rc = begin(c);
    if (rc) return rc;
    if (!valid_layer(c, layer) || !distinct_slots(c, n, slots)) return KVRT_EINVAL;
    const kvrt_layer_spec &s = c->layers[layer].spec;
    if (s.dtype != KVRT_BF16) return KVRT_EINVAL;
    const int D = s.head_dim, hkv = s.kv_heads;
    if (!tensor_ok(q, KVRT_BF16, 4) || !tensor_ok(out, KVRT_BF16, 4) || !is_contiguous(q) || !is_contiguous(out))
        return KVRT_EINVAL;
    const int64_t hq = q->dims[1], qn = q->dims[2];
    if (q->dims[0] != n || q->dims[3] != D || hq <= 0 || hq % hkv != 0 || qn <= 0 || qn > c->cfg.capacity)
        return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (out->dims[i] != q->dims[i]) return KVRT_EINVAL;
    const int group = (int)(hq / hkv);
    if (!std::isfinite(scale)) return KVRT_EINVAL;
    uint64_t tile_keys = 0;
    int64_t block_keys = 0;  // most keys any 16-query block sees
    for (int i = 0; i < n; ++i) {
        const int L = c->len_at(slots[i], layer);
        if (L < qn) return KVRT_ESTATE;
        // the oldest key any query of the chunk can see
        const int oldest = s.window > 0 ? std::max<int64_t>(0, L - qn - s.window + 1) : 0;
        if (s.layout == KVRT_LAYOUT_RING && (L - oldest > s.ring_rows || oldest < c->ring_floor(slots[i], layer)))
            return KVRT_ESTATE;
        if (s.layout == KVRT_LAYOUT_PAGED && oldest < c->first_live[slots[i]] * c->cfg.block_size) return KVRT_ESTATE;
        for (int64_t q0 = 0; q0 < qn; q0 += 16) {
            const int64_t kend = L - qn + std::min<int64_t>(qn, q0 + 16);
            const int64_t kstart = s.window > 0 ? std::max<int64_t>(0, L - qn + q0 - s.window + 1) : 0;
            tile_keys += (uint64_t)(kend - kstart);
            block_keys = std::max<int64_t>(block_keys, kend - kstart);
        }
    }
    PrefillArgs a{};
    a.kv = make_view(c, layer);
    a.len = make_len(c, layer);
    a.q = static_cast<const uint16_t *>(q->data);
    a.out = static_cast<uint16_t *>(out->data);
    a.err = c->d_err;
    a.n_items = n;
    a.group = group;
    a.qn = (int)qn;
    a.window = s.window;
    // q heads per workgroup: the largest divisor of the group up to 8 at
    // D 512 and up to 4 below (each further part of the group stages the K/V
    // tiles again, but at D <= 256 twice the workgroups of 4 heads fill more
    // of the chip: thinker sliding Q 291 44.0 -> 40.2 us, Q 2048 112.8 ->
    // 107.1 us; at D 512 four heads per workgroup take 1.9x as long);
    // KVRT_PF_HEADS_PER_WG lowers the cap
    static const int hw_env = env_int("KVRT_PF_HEADS_PER_WG", kPfMaxHeads);
    const int hw_cap = std::min(hw_env, D <= 256 ? 4 : kPfMaxHeads);
    int hw = 1;
    for (int d = 1; d <= std::min({group, kPfMaxHeads, hw_cap}); ++d)
        if (group % d == 0) hw = d;
    a.heads_per_wg = hw;
    // Key parts: up to 8 waves per workgroup, hw heads x key_parts waves each
    // splitting every tile's keys (the tile buffers bound the parts: 2 at
    // D 256, 4 below, 1 at D 512; a ring needs a tile's keys to wrap at most
    // once). More waves on each query block shorten the latency-bound chain
    // of tiles of a short chunk: 2 parts took thinker sliding Q 291 from 36.9
    // to 29.6 us, talker Q 512 from 33.6 to 29.7 us and thinker Q 2048 from
    // 93.2 to 67.2 us; 4 parts (talker: 147 KB of LDS, one workgroup per CU)
    // 43.9 us for the talker. KVRT_PF_KEY_PARTS caps it.
    static const int parts_env = env_int("KVRT_PF_KEY_PARTS", 0);
    const int64_t wgs_grid = (int64_t)((qn + 15) / 16) * hkv * (group / hw) * n;
    int parts = std::min({parts_env > 0 ? parts_env : 2, prefill_max_parts(D), 8 / hw});
    // a grid of two workgroups per CU needs no more waves per block (talker
    // Q 512: 23.3 us with one part, 24.4 us with two); KVRT_PF_KEY_PARTS
    // sets the parts there too
    if (wgs_grid >= 512 && parts_env == 0) parts = 1;
    parts = parts >= 4 ? 4 : parts >= 2 ? 2 : 1;
    while (parts > 1 && s.layout == KVRT_LAYOUT_RING && s.ring_rows < kPfKeys * parts) parts /= 2;
    a.key_parts = parts;
    // LDS DMA ring (bf16 CONTIG / RING, D 128 / 256) instead of tiles staged
    // through registers: KVRT_PF_RING = 1 / 0 forces it on / off
    static const int ring_env = [] {
        const char *e = std::getenv("KVRT_PF_RING");
        return e && *e ? std::atoi(e) : -1;
    }();
    const bool ring_default = D == 128;
    a.ring_groups = 0;
    if ((ring_env > 0 || (ring_env < 0 && ring_default)) && prefill_ring_ok(D, s.layout, parts, kPfRingGroups) &&
        (s.layout != KVRT_LAYOUT_RING || s.ring_rows >= kPfKeys))
        a.ring_groups = kPfRingGroups;
    // Talker-sized grids (>= 512 workgroups) on the ring at head_dim 128: two
    // 16-query blocks per workgroup share its staged tiles, and with the LDS
    // and waves this frees each block's keys go to two waves (talker Q 512:
    // 22.1 -> 21.3 us; pairs with one key part were 2-5% faster than single
    // blocks, four key parts without pairs took 40.0 us). KVRT_PF_QBLOCKS =
    // 1 / 2 forces single blocks / pairs; KVRT_PF_KEY_PARTS sets the parts.
    static const int qblocks_env = env_int("KVRT_PF_QBLOCKS", 0);
    a.q_blocks = 1;
    if (a.ring_groups && (qblocks_env == 2 || (qblocks_env == 0 && wgs_grid >= 512))) {
        int p2 = parts_env > 0 ? parts : 2;
        while (p2 > 1 && (hw * p2 * 2 > 8 || (s.layout == KVRT_LAYOUT_RING && s.ring_rows < kPfKeys * p2))) p2 /= 2;
        if (hw * p2 * 2 <= 8 && prefill_ring_ok(D, s.layout, p2, a.ring_groups, 2)) {
            a.q_blocks = 2;
            parts = p2;
            a.key_parts = parts;
        }
    }
    // Key split: when the query blocks give fewer than 128 workgroups (a short
    // chunk over a long context: thinker full layers, Q 291 over 2048 keys,
    // 76 workgroups on 256 CUs), each block's keys are cut into n_ksplit
    // ranges of >= 256 keys, as many as keep the grid within 256 workgroups
    // (one round: a D 512 workgroup holds 135 KB of LDS, one per CU); a merge
    // kernel then combines the ranges' partials. Q 291 at D 512: 213.8 us
    // unsplit, 134.8 / 106.1 / 142.4 / 125.7 us with 2 / 3 / 4 / 6 ranges
    // (4 ranges: 304 workgroups, a second round).
    // Not inside a capture that would need a larger workspace.
    // KVRT_PF_KSPLIT=1 turns it off, n >= 2 forces n ranges.
    static const int ksplit_env = env_int("KVRT_PF_KSPLIT", 0);
    a.n_ksplit = 1;
    const int64_t wgs1 = (int64_t)((qn + 15) / 16) * hkv * (group / hw) * n;
    if (ksplit_env != 1 && (ksplit_env > 1 || wgs1 < 128) && block_keys >= 512) {
        const int64_t want = ksplit_env > 1 ? ksplit_env : std::min<int64_t>(256 / wgs1, block_keys / 256);
        const int nks = (int)std::max<int64_t>(1, std::min<int64_t>(want, 16));
        const size_t po = ((size_t)n * hq * qn * nks * D + 63) / 64 * 64;
        const size_t bytes = po * 4 + (size_t)n * hq * qn * nks * 8 + 256;
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        const bool capturing = hipStreamIsCapturing(c->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
        if (nks > 1 && (bytes <= c->ws_bytes || (!capturing && ensure_workspace(c, bytes) == KVRT_OK))) {
            a.n_ksplit = nks;
            a.part_o = c->ws;
            a.part_ml = reinterpret_cast<float2 *>(c->ws + po);
        }
        if (c->poisoned) return KVRT_EDEVICE;
    }
    a.pmask = launch_masks(c, n, slots);
    a.scale_log2 = scale * 1.4426950408889634f;
    for (int i = 0; i < n; ++i) a.slots[i] = slots[i];
    c->counters.launches += a.n_ksplit > 1 ? 2 : 1;
    if (launch_prefill(a, D, enq(c)) != hipSuccess) return poison(c);
    c->counters.attended_keys += tile_keys * hkv;
    c->counters.attended_bytes += tile_keys * hkv * (uint64_t)D * 2 * 2;
    return KVRT_OK;
}

int kvrt_attend_tensors_async(const kvrt_tensor *q, const kvrt_tensor *k, const kvrt_tensor *v,
                              const int32_t *device_lengths, const kvrt_tensor *prefix_attention,
                              const kvrt_tensor *out, float scale, int32_t window, void *stream) {
    TensorCall tc;
    int rc = tensor_call_setup(q, k, v, device_lengths, prefix_attention, out, scale, window, target_wgs(kvrt_config{}),
                               tc);
    if (rc != KVRT_OK) return rc;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    std::lock_guard<std::mutex> lock(g_tensor_mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return KVRT_EDEVICE;
    TensorWorkspace &ws = g_tensor_ws[{dev, st}];
    if (ws.bytes < tc.bytes) {
        // no allocation inside a stream capture: an eager call of the largest
        // shape sizes the workspace first
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) return KVRT_EDEVICE;
        if (cs != hipStreamCaptureStatusNone) return KVRT_ESTATE;
        float *fresh = nullptr;
        const size_t want = std::max(tc.bytes, (size_t)1 << 20);
        if (hipMalloc(&fresh, want) != hipSuccess) return KVRT_EDEVICE;
        // the error flag and the arrival counters start at zero
        if (launch_zero(fresh, kTensorWsParts * 4, st) != hipSuccess) return KVRT_EDEVICE;
        if (ws.ptr) g_tensor_retired.push_back(ws.ptr);
        ws.ptr = fresh;
        ws.bytes = want;
    }
    return tensor_call_launch(tc, ws.ptr, st, true);
}

int kvrt_attend_tensors_noalloc_async(const kvrt_tensor *q, const kvrt_tensor *k, const kvrt_tensor *v,
                                      const int32_t *device_lengths, const kvrt_tensor *prefix_attention,
                                      const kvrt_tensor *out, float scale, int32_t window, void *stream) {
    // the split count of kvrt_attend_tensors_async, halved until the partials
    // fit the scratch (one workgroup per (item, kv head) at the least)
    int target = target_wgs(kvrt_config{});
    TensorCall tc;
    int rc = tensor_call_setup(q, k, v, device_lengths, prefix_attention, out, scale, window, target, tc);
    if (rc != KVRT_OK) return rc;
    while (tc.bytes > kScratchBytes && target > 1) {
        target /= 2;
        tc = TensorCall{};
        rc = tensor_call_setup(q, k, v, device_lengths, prefix_attention, out, scale, window, target, tc);
        if (rc != KVRT_OK) return rc;
    }
    if (tc.bytes > kScratchBytes) return KVRT_EINVAL;  // beyond KVRT_NOALLOC_SCRATCH_BYTES
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return KVRT_EDEVICE;
    float *ws = nullptr;
    rc = scratch_pointer(dev, &ws);
    if (rc != KVRT_OK) return rc;
    // the merge kernel after the decode: the scratch holds no arrival counters
    return tensor_call_launch(tc, ws, static_cast<hipStream_t>(stream), false);
}

int kvrt_tensors_status(void *stream) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    std::lock_guard<std::mutex> lock(g_tensor_mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return KVRT_EDEVICE;
    auto it = g_tensor_ws.find({dev, st});
    if (it == g_tensor_ws.end() || !it->second.ptr) return KVRT_OK;
    if (hipStreamSynchronize(st) != hipSuccess) return KVRT_EDEVICE;
    int32_t err = 0;
    if (hipMemcpy(&err, it->second.ptr, sizeof(err), hipMemcpyDeviceToHost) != hipSuccess) return KVRT_EDEVICE;
    if (err == 0) return KVRT_OK;
    if (launch_zero(it->second.ptr, kTensorWsHead * 4, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
        return KVRT_EDEVICE;
    return KVRT_EFAULT;
}

int kvrt_copy_rows_async(const kvrt_tensor *src, const kvrt_tensor *dst, int64_t rows, void *stream) {
    if (!src || !dst || !src->data || !dst->data || src->ndim != 4 || dst->ndim != 4 || src->dtype != dst->dtype)
        return KVRT_EINVAL;
    const int es = elem_size(src->dtype);
    if (es != 2 && es != 4) return KVRT_EINVAL;
    if (src->strides[3] != 1 || dst->strides[3] != 1) return KVRT_EINVAL;
    for (int i = 0; i < 4; ++i)
        if (i != 2 && src->dims[i] != dst->dims[i]) return KVRT_EINVAL;
    if (rows < 0 || rows > src->dims[2] || rows > dst->dims[2]) return KVRT_EINVAL;
    const int64_t row_bytes = src->dims[3] * es;
    if (row_bytes % 4 != 0 || (reinterpret_cast<uintptr_t>(src->data) & 3u) ||
        (reinterpret_cast<uintptr_t>(dst->data) & 3u))
        return KVRT_EINVAL;
    CopyRowsArgs a{};
    a.src = static_cast<const uint8_t *>(src->data);
    a.dst = static_cast<uint8_t *>(dst->data);
    a.d0 = src->dims[0];
    a.d1 = src->dims[1];
    a.rows = rows;
    a.row_bytes = row_bytes;
    a.s0 = src->strides[0] * es;
    a.s1 = src->strides[1] * es;
    a.sr = src->strides[2] * es;
    a.t0 = dst->strides[0] * es;
    a.t1 = dst->strides[1] * es;
    a.tr = dst->strides[2] * es;
    if ((a.s0 | a.s1 | a.sr | a.t0 | a.t1 | a.tr) & 3) return KVRT_EINVAL;
    return launch_copy_rows(a, static_cast<hipStream_t>(stream)) == hipSuccess ? KVRT_OK : KVRT_EDEVICE;
}

int kvrt_session_state(kvrt_ctx *c, int32_t slot, int32_t layer, int32_t *length) {
    if (!c || !length || !valid_slot(c, slot) || !valid_layer(c, layer)) return KVRT_EINVAL;
    *length = c->len_at(slot, layer);
    return KVRT_OK;
}

int kvrt_sync_lengths(kvrt_ctx *c) {
    if (!c) return KVRT_EINVAL;
    if (c->poisoned) return KVRT_EPOISONED;
    if (hipSetDevice(c->device) != hipSuccess) return poison(c);
    if (hipStreamSynchronize(c->stream) != hipSuccess) return poison(c);
    c->dirty = false;
    std::vector<int32_t> dev(c->len.size());
    if (hipMemcpy(dev.data(), c->d_len, dev.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return poison(c);
    for (size_t i = 0; i < dev.size(); ++i) {
        if (dev[i] < 0 || dev[i] > c->cfg.capacity) return KVRT_EFAULT;
    }
    c->len = dev;
    for (int slot = 0; slot < c->cfg.n_slots; ++slot)
        for (int l = 0; l < c->cfg.n_layers; ++l)
            if (c->layers[l].owner == l) c->ring_advance(slot, l);
    c->lens_stale = false;
    return KVRT_OK;
}

int kvrt_get_counters(kvrt_ctx *c, kvrt_counters *out) {
    if (!c || !out) return KVRT_EINVAL;
    *out = c->counters;
    return KVRT_OK;
}

int kvrt_health(kvrt_ctx *c) {
    if (!c) return KVRT_EINVAL;
    if (c->poisoned) return KVRT_EPOISONED;
    if (hipSetDevice(c->device) != hipSuccess) return poison(c);
    if (hipStreamSynchronize(c->stream) != hipSuccess) return poison(c);
    c->dirty = false;
    int32_t err = 0;
    if (hipMemcpy(&err, c->d_err, sizeof(err), hipMemcpyDeviceToHost) != hipSuccess) return poison(c);
    if (err != 0) return KVRT_EFAULT;
    return KVRT_OK;
}

int kvrt_debug_inject_failure(kvrt_ctx *c) {
    if (!c) return KVRT_EINVAL;
    c->inject = true;
    return KVRT_OK;
}

}  // extern "C"

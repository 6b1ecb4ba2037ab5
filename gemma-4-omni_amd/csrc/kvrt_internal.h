// kvrt_internal.h — launch argument blocks shared by the host runtime
// (kvrt_runtime.hip) and the kernels (kvrt_kernels.hip).
//
// Every block is passed BY VALUE as the kernel argument (kernarg segment),
// so a launch captures its own copy of slot lists and page-table edits at
// enqueue time; nothing the host changes afterwards can race the kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kvrt.h"

namespace kvrt {

constexpr int kMaxItems = KVRT_MAX_ITEMS;
constexpr int kWaves = 4;            // waves per attention workgroup
constexpr int kPtUpdates = 128;      // page-table edits carried by one launch
constexpr int kMaxPositions = KVRT_MAX_POSITIONS;  // explicit positions carried by one write
constexpr int kMaxInt8Rows = 8;      // query rows per kv head of an INT8 decode (g * Q)

// Key-row groups a decode wave keeps in flight per main-loop pass, by row
// tile R: all of them are loaded before the first is used, so a wave has
// U * 2 KiB (bf16: K and V, 16 B per lane) outstanding; fewer for larger R,
// whose query rows and accumulators take the registers (8 rows: 3 groups,
// 182 VGPRs — lighter on a concurrently running stream than 4).
#ifndef KVRT_UNROLL8
#define KVRT_UNROLL8 3
#endif
constexpr int keys_unroll(int R) { return R <= 4 ? 8 : (R == 8 ? KVRT_UNROLL8 : 2); }

// bf16 CONTIG / RING decodes of <= 4 rows per kv head stream K/V straight
// into LDS (global_load_lds_dwordx4) through a ring of kDmaStages stages of
// dma_unroll(R) key groups per wave, so the next stages stay in flight while a
// wave computes on the current one without holding registers for them.
// 4 groups x 2 stages (68 KB of LDS per workgroup) give the shortest
// two-stream step with the single-launch decode (3, 5 and 6 groups measured).
#ifndef KVRT_DMA_UNROLL
#define KVRT_DMA_UNROLL 4
#endif
#ifndef KVRT_DMA_STAGES
#define KVRT_DMA_STAGES 2
#endif
#ifndef KVRT_DECODE_DMA
#define KVRT_DECODE_DMA 1
#endif
#ifndef KVRT_DMA_MAX_ROWS
#define KVRT_DMA_MAX_ROWS 4
#endif
#ifndef KVRT_DMA_UNROLL8
#define KVRT_DMA_UNROLL8 2
#endif
constexpr int kDmaStages = KVRT_DMA_STAGES;
// Key groups per ring stage (8-row tiles hold more q rows and accumulators).
constexpr int dma_unroll(int R) { return R <= 4 ? KVRT_DMA_UNROLL : KVRT_DMA_UNROLL8; }
// Bytes of one wave's ring: q rows (ceil(R * D/8 / 64) KiB) + stages x groups x (K, V).
constexpr int dma_wave_bytes(int R, int head_dim) {
    return (kDmaStages * dma_unroll(R) * 2 + (R * (head_dim / 8) + 63) / 64) * 1024;
}
// The rings of a workgroup fit gfx950's 160 KiB of LDS with 1 KiB left for
// the merge's (m, l) table (an M0-addressed LDS DMA reaches the whole range:
// probed at byte 96 KiB of a 128 KiB allocation); a wave's fp32 partial
// (R x D) must fit its own ring.
// (int8 PAGED decodes measured no faster through such a ring — 28.2 vs
// 28.0 us at config 5's layer, a 256-byte block of scales per stage, 4
// workgroups per CU — and load their passes into registers.)
constexpr bool decode_dma(int R, int dtype, int layout, int head_dim) {
    return KVRT_DECODE_DMA && dtype == KVRT_BF16 && layout != KVRT_LAYOUT_PAGED && R <= KVRT_DMA_MAX_ROWS &&
           kWaves * dma_wave_bytes(R, head_dim) <= 160 * 1024 - 1024 &&
           R * head_dim * 4 <= dma_wave_bytes(R, head_dim);  // the wave's partial fits its drained ring
}
// int8 decodes are VALU-bound (a dequantise and R FMAs per value): 2 key
// groups per pass keep them at 118 VGPRs, 4 waves per SIMD.
#ifndef KVRT_INT8_UNROLL
#define KVRT_INT8_UNROLL 2
#endif
// Key groups per main-loop pass of decode_kernel.
constexpr int decode_unroll(int R, int dtype, int layout, int head_dim) {
    return decode_dma(R, dtype, layout, head_dim) ? dma_unroll(R)
           : dtype == KVRT_INT8 ? KVRT_INT8_UNROLL : keys_unroll(R);
}

// Where the rows of one layer live. Row (slot, head, pos) starts at element
//   CONTIG: slot*slot_stride + head*head_stride + pos*row_stride
//   RING:   slot*slot_stride + head*head_stride + (pos % rows)*row_stride
//   PAGED:  ((page*kv_heads + head)*rows + pos % rows)*D, page = pt[slot][pos / rows]
// INT8 scales are indexed by the same row number (element offset / D).
struct KVView {
    void *k;
    void *v;
    float *ks;
    float *vs;
    int64_t slot_stride;
    int64_t head_stride;
    int64_t row_stride;
    int32_t rows;        // CONTIG: capacity, RING: ring rows, PAGED: block size
    int32_t layout;
    int32_t kv_heads;
    int32_t block_shift; // PAGED: log2(block size)
    int32_t *page_table; // PAGED: [n_slots, pt_stride]
    int32_t pt_stride;
    int32_t pool_pages;
};

struct Lengths {
    int32_t *lens;   // device lengths; entry = lens[slot*stride + offset]
    int32_t stride;
    int32_t offset;
};

// Prefix-attention mask of one slot (device, 128 B): key position k < len is
// visible only if bit k of bits is set; bits at or past len are set. A
// decode wave keeps word (lane & 15) in a register and finds the word of a
// key with a lane shuffle.
constexpr int kPrefixWords = KVRT_MAX_PREFIX_MASK / 32;
struct PrefixMask {
    int32_t len;
    int32_t pad[15];
    uint32_t bits[kPrefixWords];
};
static_assert(sizeof(PrefixMask) == 128, "prefix mask record");

// Packs n masks (int64 / int32 / bool elements, [n, P] with element strides)
// into PrefixMask records dst[index[i]].
struct PrefixPackArgs {
    const uint8_t *src;
    int64_t item_stride;   // elements
    int32_t elem_bytes;    // 8, 4 or 1
    int32_t n_items;
    int32_t plen;          // P
    PrefixMask *dst;
    int32_t index[kMaxItems];
};

struct AppendArgs {
    KVView kv;
    Lengths len;
    const uint16_t *k_src;  // bf16 [n, kv_heads, rows, D] (strided)
    const uint16_t *v_src;
    int64_t src_item_stride;
    int64_t src_head_stride;
    int64_t src_row_stride;
    int32_t n_items;
    int32_t rows;           // Q (append) or S (import)
    int32_t import_mode;    // 0: pos0 = device length, length += rows
                            //    (one workgroup per item: graph-replay safe)
                            // 1: pos0 = base_pos (host), length = base_pos + rows
                            //    (any grid: nothing reads the length)
                            // 2: row r of item i at pos[i*rows + r],
                            //    length = max(length, pos_end[i])
    int32_t base_pos;       // mode 1: position of row 0
    int32_t keep_from;      // mode 1: rows below this position are not stored
    int32_t *err;           // device error flag
    int32_t n_upd;          // page-table edits applied before the writes
    int32_t upd_idx[kPtUpdates];
    int32_t upd_val[kPtUpdates];
    int32_t pos[kMaxPositions];   // mode 2 only
    int32_t pos_end[kMaxItems];   // mode 2 only: max position + 1 per item
    int32_t slots[kMaxItems];
};

struct GatherArgs {
    KVView kv;
    Lengths len;
    void *out_k;            // [n, kv_heads, lmax, D] bf16 or fp32
    void *out_v;
    int64_t out_item_stride, out_head_stride, out_row_stride;
    void *mask;             // [n, lmax] or null
    int64_t mask_item_stride;
    int32_t mask_dtype;
    int32_t out_fp32;
    int32_t n_items;
    int32_t lmax;
    int32_t window;         // ring default start rule
    int32_t has_start;
    int32_t *err;
    // fused append (bf16 CONTIG / RING; else null): k_new, v_new [n, kv_heads,
    // qn, D] contiguous land at each item's device length before the gather
    // reads, and the last workgroup of an item (arrival count in cnt) advances
    // that length by qn
    const uint16_t *k_new;
    const uint16_t *v_new;
    uint32_t *cnt;
    int32_t qn;
    int32_t start[kMaxItems];
    int32_t slots[kMaxItems];
};

struct DecodeArgs {
    KVView kv;
    Lengths len;
    const uint16_t *q;      // [n, Hq, Q, D] contiguous
    uint16_t *out;          // [n, Hq, Q, D] contiguous
    const uint16_t *k_new;  // fused append: [n, kv_heads, Q, D] contiguous, else null
    const uint16_t *v_new;
    float *part_acc;        // [n, kv_heads, n_split, R, D]
    float2 *part_ml;        // [n, kv_heads, n_split, R]
    int32_t *err;
    int32_t n_items;
    int32_t group;          // Hq / kv_heads
    int32_t qn;             // Q
    int32_t window;
    int32_t n_split;        // wave splits per (item, kv head) = gridDim.x * kWaves
    int32_t advance;        // the merge kernel adds qn to each item's length
    int32_t n_parts;        // partials per (item, kv head) the merge kernel combines
    uint32_t *cnt;          // non-null: the decode merges its own partials (see kCntItems)
    const PrefixMask *pmask;  // non-null: prefix-attention masks, indexed by slot
    uint8_t order[kMaxItems];  // PAGED: item of grid z-index i, the most visible keys first
    float scale_log2;       // softmax scale * log2(e)
    // PAGED fused appends: page-table edits page_table[upd_idx[i]] = upd_val[i]
    // that map the new rows' pages (a slot's rows crossing into a new block).
    // The launch's first workgroup writes them into the table; no workgroup of
    // the launch reads those entries (the new rows come from k_new / v_new),
    // and the workgroups storing the new rows take their page from here.
    int32_t n_upd;
    int32_t upd_idx[kMaxItems];
    int32_t upd_val[kMaxItems];
    int32_t slots[kMaxItems];
};

// Arrival counters of the single-launch decode, per context: one per (item,
// kv head) at item * kv_heads + kvh, then one per item at kCntItemBase + item.
// Every launch leaves them at zero.
constexpr int kCntItemBase = kMaxItems * 64;
// The fused append + gather counts its workgroups' arrivals per (item, kv
// head), then per item, each counter on a 128-byte line of its own: up to
// hundreds of workgroups arrive per item, and atomics on one line serialise
// (all items' counters on one line made the launch ~7 us longer).
constexpr int kCntLineWords = 32;
constexpr int kCntGatherBase = kCntItemBase + kMaxItems + kCntLineWords;  // line aligned below
constexpr int kCntGatherHead(int item, int h) {
    return (kCntGatherBase / kCntLineWords + item * 64 + h) * kCntLineWords;
}
constexpr int kCntGatherItem(int item) { return kCntGatherHead(kMaxItems, 0) + item * kCntLineWords; }
constexpr int kCntWords = kCntGatherItem(kMaxItems);

// The split-K decode merges its 4 waves' partials in LDS (one partial per
// workgroup) when R * D floats per wave fit.
constexpr bool decode_wg_merge(int head_dim, int rows_tile) { return rows_tile * head_dim <= 4096; }
// Row tiles that run on the MFMA decode kernel (bf16, causal / window visibility).
constexpr int kMfmaDecodeMinRows = 8;
constexpr int kMfmaDecodeKeys = 16;  // keys per MFMA decode tile
// The MFMA decode's LDS DMA ring (K and V tiles streamed into LDS, two
// stages per wave at D 128, one at D 256): bf16 CONTIG / RING tiles of 8
// rows at the head dims switched on here.
#ifndef KVRT_MFMA_DMA_D128
#define KVRT_MFMA_DMA_D128 1
#endif
#ifndef KVRT_MFMA_DMA_D256
#define KVRT_MFMA_DMA_D256 1
#endif
// int8 PAGED decodes of up to 8 rows per kv head at head_dim 64 / 128 run on
// decode_i8_mfma_kernel: 32-key tiles of int8 K, V and scales DMAd into a ring
// of KVRT_I8_MFMA_STAGES stages per wave (8.25 KiB per stage at D 128).
#ifndef KVRT_I8_MFMA
#define KVRT_I8_MFMA 1
#endif
#ifndef KVRT_I8_MFMA_STAGES
#define KVRT_I8_MFMA_STAGES 2
#endif
constexpr int kI8MfmaKeys = 32;  // keys per int8 MFMA decode tile
constexpr bool i8_mfma_dma(int head_dim, int rows_tile) {
    return KVRT_I8_MFMA && (head_dim == 64 || head_dim == 128) && rows_tile >= 1 && rows_tile <= 8;
}
constexpr bool mfma_decode_dma(int head_dim, int rows_tile, int dtype, int layout) {
    return dtype == KVRT_BF16 && layout != KVRT_LAYOUT_PAGED && rows_tile <= 8 &&
           ((head_dim == 128 && KVRT_MFMA_DMA_D128) || (head_dim == 256 && KVRT_MFMA_DMA_D256));
}

// Talker visibility of one item (host-validated: 0 <= prefix_start <=
// prefix_pos < audio_start <= audio_pos < length). Query row i of the item is
// the audio query when i == Q - 1, the prefix query otherwise (Q = 2).
//   prefix query: keys [0, max(prefix_pos, prefix_start - 1)]
//   audio query:  keys [0, prefix_start) U [prefix_start, prefix_pos] (mode != 1)
//                      U [audio_start, audio_pos]
// and in mode 2 the audio query's score of a key in [prefix_start, prefix_pos]
// gets gate_log2 added (log2 domain).
struct TalkerItem {
    int32_t prefix_start;
    int32_t prefix_pos;
    int32_t audio_start;
    int32_t audio_pos;
    int32_t mode;
    float gate_log2;
};

struct TalkerArgs : DecodeArgs {
    TalkerItem talk[kMaxItems];
};

struct PrefillArgs {
    KVView kv;
    Lengths len;
    const uint16_t *q;      // [n, Hq, Q, D] contiguous
    uint16_t *out;          // [n, Hq, Q, D] contiguous
    int32_t *err;
    int32_t n_items;
    int32_t group;          // Hq / kv_heads (waves per workgroup)
    int32_t qn;             // Q (query rows per item)
    int32_t window;
    int32_t heads_per_wg;   // q heads of the group served by one workgroup (divides group)
    int32_t key_parts;      // waves per head splitting every tile's keys (1, 2 or 4)
    int32_t ring_groups;    // > 0: LDS DMA ring of key_parts * ring_groups 32-key stages (prefill_ring_ok)
    int32_t q_blocks;       // 16-query blocks per workgroup sharing its staged tiles (1; 2 on the ring)
    int32_t n_ksplit;       // key ranges per query block; > 1: partials to part_o / part_ml
    float *part_o;          // [n, Hq, Q, n_ksplit, D] unnormalised outputs
    float2 *part_ml;        // [n, Hq, Q, n_ksplit] (running max in log2 units, sum)
    const PrefixMask *pmask;  // non-null: prefix-attention masks, indexed by slot
    float scale_log2;
    int32_t slots[kMaxItems];
};

// Edits lens[idx[i]] = val[i]. With check set (a rollback), all of them or
// none: only when every lens[idx[i]] still holds expect[i], the value the
// host validated against; otherwise err[0] is raised and nothing changes.
struct SetLenArgs {
    int32_t *lens;
    int32_t n;
    int32_t check;
    int32_t *err;
    int32_t idx[kPtUpdates];
    int32_t val[kPtUpdates];
    int32_t expect[kPtUpdates];
};

// Static description of one layer, kept in device memory by the context
// (uploaded at create and when a RoPE table is set); read by the
// slot-lifecycle kernels, which may span every layer of a context.
struct LayerDesc {
    KVView kv;
    int32_t head_dim;
    int32_t dtype;
    float rope_scaling;
    int32_t rope_pairs;       // entries of inv_freq (head_dim / 2), 0 = keys not rotated
    const float *inv_freq;    // device [head_dim / 2] or null
};

constexpr int kMaxMoveLayers = 64;   // layer entries per slot-move launch
constexpr int kMaxRebaseRows = 128;  // rows one rebase workgroup holds in registers

// Row moves between slots (and contexts) of identically shaped layers:
// entry e moves rows[e] positions of every kv head of layer[e] from
// (src_slot, src_pos0[e] + r) to (dst_slot, dst_pos0[e] + r).
struct SlotMoveArgs {
    const LayerDesc *src;     // device table of the source context
    const LayerDesc *dst;     // device table of the destination context
    int32_t *err;
    int32_t src_slot;
    int32_t dst_slot;
    int32_t n_entries;
    int32_t rope_delta;       // rebase: moved keys rotate by this many positions
    int32_t layer[kMaxMoveLayers];
    int32_t src_pos0[kMaxMoveLayers];
    int32_t dst_pos0[kMaxMoveLayers];
    int32_t rows[kMaxMoveLayers];
};

struct CopyRowsArgs {
    const uint8_t *src;
    uint8_t *dst;
    int64_t d0, d1, rows, row_bytes;          // row_bytes multiple of 4
    int64_t s0, s1, sr;                       // src strides in bytes
    int64_t t0, t1, tr;                       // dst strides in bytes
};

// ---- launchers (kvrt_kernels.hip) ----------------------------------------
hipError_t launch_append(const AppendArgs &a, int head_dim, int dtype, int grid_x, hipStream_t s);
hipError_t launch_gather(const GatherArgs &a, int head_dim, int dtype, hipStream_t s);
// Split-K attention over the view, then the merge kernel.
hipError_t launch_decode(const DecodeArgs &a, int head_dim, int dtype, int rows_per_head,
                         hipStream_t s);
// The same decode with S and P.V on MFMA (bf16, row tiles 8 and 16), one
// partial per workgroup; then the merge kernel.
hipError_t launch_decode_mfma(const DecodeArgs &a, int head_dim, int dtype, int rows_per_head, hipStream_t s);
// The same split-K decode under the talker visibility (bf16 CONTIG layers).
hipError_t launch_decode_talker(const TalkerArgs &a, int head_dim, int rows_per_head, hipStream_t s);
// Chunked-prefill attention on MFMA (bf16 CONTIG / RING / PAGED layers).
hipError_t launch_prefill(const PrefillArgs &a, int head_dim, hipStream_t s);
// Most q heads one prefill workgroup computes (one wave each); a larger GQA
// group is served by several workgroups.
constexpr int kPfMaxHeads = 8;
// Most waves per head (key parts) a prefill workgroup's tile buffers allow:
// each part needs its own 32-key sub-tile, double-buffered in LDS.
constexpr int kPfKeys = 32;  // keys per LDS sub-tile of the prefill kernel
constexpr int prefill_max_parts(int head_dim) { return head_dim >= 512 ? 1 : head_dim >= 256 ? 2 : 4; }
// Shapes of the prefill's LDS DMA ring: bf16 CONTIG / RING rows of 128 or
// 256 dims, key_parts (1 or 2) * kPfRingGroups unpadded 32-key stages (K and
// V), one group of key_parts stages computed while the next is in flight
// (deeper rings measured slower: their LDS costs workgroups per CU); at
// head_dim 128 one or two 16-query blocks per workgroup.
constexpr int kPfRingGroups = 2;
constexpr bool prefill_ring_ok(int head_dim, int layout, int key_parts, int groups, int q_blocks = 1) {
    return (head_dim == 128 || head_dim == 256) && layout != KVRT_LAYOUT_PAGED && groups == kPfRingGroups &&
           (key_parts == 1 || key_parts == 2) && key_parts * groups * 32 * head_dim * 2 * 2 <= 128 * 1024 &&
           (q_blocks == 1 || (q_blocks == 2 && head_dim == 128));
}
hipError_t launch_set_lens(const SetLenArgs &a, hipStream_t s);
hipError_t launch_set_pages(int32_t *pt, int n, const int32_t *idx, const int32_t *val,
                            hipStream_t s);
hipError_t launch_copy_rows(const CopyRowsArgs &a, hipStream_t s);
// Copy between two slots (any layout, bf16 or int8 with scales); ranges must not overlap.
hipError_t launch_slot_copy(const SlotMoveArgs &a, int64_t max_units, hipStream_t s);
// In-place move of <= kMaxRebaseRows rows per entry within one slot, keys
// rotated by rope_delta positions where the layer has a RoPE table (bf16).
hipError_t launch_slot_rebase(const SlotMoveArgs &a, int max_heads, hipStream_t s);
hipError_t launch_zero(void *p, uint64_t bytes, hipStream_t s);
hipError_t launch_prefix_pack(const PrefixPackArgs &a, hipStream_t s);

// Smallest instantiated row tile >= rows (1, 2, 4, 8, 16); 0 if too large.
int rows_tile(int rows);
// Keys one wave consumes per main-loop iteration of decode_kernel.
int keys_per_iteration(int head_dim, int rows_tile, int dtype, int layout);

}  // namespace kvrt

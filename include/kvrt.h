/*
 * kvrt.h — C ABI of the MI355X (gfx950) KV-cache runtime.
 *
 * One shared library, libkvrt.so, holds the hand-written HIP kernels for the
 * per-frame KV hot path of the duplex decode loops (Gemma-4-E2B-shaped
 * thinker/listener, Qwen3-TTS-shaped talker):
 *
 *   append  (contiguous, sliding-window ring, paged bf16 / paged int8)
 *   gather  (ragged N-stream micro-batch -> padded [N, H, Lmax, D] + mask)
 *   truncate / evict (turn-local rollback as length / page-table edits)
 *   attend  (GQA split-K decode attention, fp32 softmax and accumulators)
 *
 * Conventions (mirroring the reference native ABIs, e.g.
 * native/gemma4_listener_microbatch/gemma4_listener.h:36-50 and
 * native/qwen_talker/qwen_talker.h:55-68):
 *   - every entry point is extern "C" and returns int: 0 ok, negative error
 *     class (see KVRT_E*). Argument errors leave the context untouched.
 *   - a failed device enqueue poisons the context; a poisoned context
 *     refuses every later mutating call with KVRT_EPOISONED.
 *   - host descriptors (kvrt_tensor, arrays of slot ids) are read
 *     synchronously during the call and never retained.
 *   - device payloads (queries, new K/V rows, outputs) are caller-owned and
 *     borrowed for the duration of the enqueued work; KV storage is owned by
 *     the context unless the caller binds its own storage at create time.
 *   - every mutating call is asynchronous on the stream bound with
 *     kvrt_bind_stream (default: the null stream). A context stays on its
 *     bound stream: binding another one is refused while work enqueued by the
 *     context may still run (see kvrt_bind_stream). Lengths are tracked on the
 *     host (authoritative, used for validation) and mirrored in device memory
 *     where the kernels read them.
 *   - one owner host thread per context; calls on one context are not
 *     thread-safe (the Python binding asserts its creating thread).
 *   - every slot carries a generation, renewed whenever the slot's contents
 *     are replaced (reset, clone / copy into it); the lifecycle calls take
 *     the generation the caller last saw and refuse a stale one.
 *
 * Stream handles are passed as void* (a hipStream_t) so that the header
 * needs no HIP or torch types.
 */
#ifndef KVRT_H
#define KVRT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVRT_ABI_VERSION 3u
#define KVRT_MAX_RANK 4
#define KVRT_MAX_ITEMS 64      /* slots per batched call                 */
#define KVRT_MAX_POSITIONS 128 /* rows per kvrt_write_positions_async call */
#define KVRT_MAX_ROLLOVER_ROWS 128 /* rows kept by one kvrt_rollover_async    */
#define KVRT_MAX_PREFIX_MASK 512   /* positions a prefix-attention mask covers  */
#define KVRT_ANY_GENERATION 0ull   /* expected_generation: skip the slot check  */

/* ---- return codes ------------------------------------------------------ */
#define KVRT_OK 0
#define KVRT_EINVAL (-1)    /* invalid argument, shape, dtype or slot id      */
#define KVRT_ESTATE (-2)    /* state mismatch: capacity, rollback beyond ring */
#define KVRT_EDEVICE (-3)   /* device enqueue/allocation failed: ctx poisoned */
#define KVRT_EPOISONED (-4) /* ctx poisoned by an earlier device failure      */
#define KVRT_ENOMEM (-5)    /* page pool exhausted                            */
#define KVRT_EFAULT (-6)    /* device-side error flag raised (health check)   */

/* ---- capability bits (kvrt_capabilities) -------------------------------- */
#define KVRT_CAP_CONTIG (1ull << 0)
#define KVRT_CAP_RING (1ull << 1)
#define KVRT_CAP_PAGED (1ull << 2)
#define KVRT_CAP_INT8 (1ull << 3)
#define KVRT_CAP_FUSED_APPEND_ATTEND (1ull << 4)
#define KVRT_CAP_GATHER (1ull << 5)
#define KVRT_CAP_DEVICE_LENGTHS (1ull << 6)
#define KVRT_CAP_TENSOR_ATTEND (1ull << 7)
#define KVRT_CAP_PREFILL_MFMA (1ull << 8)
#define KVRT_CAP_TALKER_MASK (1ull << 9)
#define KVRT_CAP_PREFIX_ATTENTION (1ull << 10)
#define KVRT_CAP_SLOT_GENERATION (1ull << 11)
#define KVRT_CAP_STREAM_CONFINED (1ull << 12)
#define KVRT_CAP_ROLLBACK_POSITION (1ull << 13) /* truncate checks expected_len; import refuses live slots */

/* ---- enums ------------------------------------------------------------- */
enum kvrt_layout {
    KVRT_LAYOUT_CONTIG = 0, /* [slots, kv_heads, capacity, D] per layer        */
    KVRT_LAYOUT_RING = 1,   /* [slots, kv_heads, ring_rows, D]; row = pos mod R */
    KVRT_LAYOUT_PAGED = 2,  /* [pool_pages, kv_heads, block, D] + page table    */
};

enum kvrt_dtype {
    KVRT_BF16 = 0,
    KVRT_INT8 = 1, /* symmetric, one fp32 scale per (token, head) */
    KVRT_FP32 = 2,
    KVRT_BOOL = 3, /* 1 byte: 0 / 1 */
    KVRT_INT32 = 4,
    KVRT_INT64 = 5,
};

/* ---- descriptors --------------------------------------------------------- */
/* Strided tensor view. Strides are in ELEMENTS; the last dimension must be
 * contiguous (stride 1) for every K/V/Q/O tensor. */
typedef struct kvrt_tensor {
    void *data;
    int32_t dtype;
    int32_t ndim;
    int64_t dims[KVRT_MAX_RANK];
    int64_t strides[KVRT_MAX_RANK];
} kvrt_tensor;

typedef struct kvrt_layer_spec {
    int32_t layout;     /* enum kvrt_layout                                   */
    int32_t dtype;      /* KVRT_BF16 or KVRT_INT8 (INT8 requires PAGED)        */
    int32_t kv_heads;   /* 1..64                                              */
    int32_t head_dim;   /* 64, 128, 256 or 512                                */
    int32_t window;     /* sliding window W (keys p-W+1..p visible), 0 = global */
    int32_t ring_rows;  /* RING only: physical rows R >= W + max_q - 1         */
    int32_t shared_src; /* -1, or an earlier layer whose K/V this layer reads  */
    int32_t reserved;
} kvrt_layer_spec;

typedef struct kvrt_config {
    uint32_t struct_size; /* sizeof(kvrt_config)                              */
    int32_t n_layers;
    int32_t n_slots;      /* sessions / streams                               */
    int32_t capacity;     /* max logical tokens per slot                      */
    int32_t block_size;   /* PAGED: tokens per page (power of two, e.g. 16)   */
    int32_t pool_pages;   /* PAGED: pages in the shared pool (< 2^24, and
                             pool_pages * kv_heads * block_size < 2^31 for
                             every PAGED layer: rows are numbered in 32 bits) */
    int32_t max_q;        /* max rows per decode append / attend; RING rows >= W + max_q - 1 */
    int32_t pool_seed;    /* PAGED: nonzero = hand out pool pages in an order
                             shuffled with this seed (0 = ascending)          */
    int32_t decode_wgs;   /* split-K decode: target workgroups per launch
                             (0 = 512, or KVRT_TARGET_WGS). Contexts whose
                             launches run beside another model's on a second
                             stream do better with fewer (e.g. 192)          */
    int32_t decode_kernel; /* KVRT_DECODE_*: which kernel runs bf16 decodes of
                             8 or 16 query rows per kv head                   */
    int32_t decode_merge;  /* KVRT_MERGE_*: how a split-K decode combines its
                             partial results                                  */
} kvrt_config;

/* kvrt_config.decode_kernel. AUTO: MFMA for bf16 decodes of 16 rows per kv
 * head, and of 8 rows at head_dim 512 or over >= 2048 visible keys; the VALU
 * kernel otherwise (int8 included). VALU / MFMA force one kernel for every
 * eligible decode (MFMA: bf16 with 8 or 16 rows per kv head, or int8 PAGED
 * with up to 8; not the talker masks; other decodes always run on the VALU
 * kernel). */
#define KVRT_DECODE_AUTO 0
#define KVRT_DECODE_VALU 1
#define KVRT_DECODE_MFMA 2

/* kvrt_config.decode_merge. A split-K decode leaves one partial (running max,
 * sum, output) per workgroup and kv head, combined by a merge step:
 * SEPARATE: a second kernel launch merges them;
 * LAST_WG: the last workgroup of each (slot, kv head) to finish merges them
 *   inside the decode launch (one launch per layer); the VALU kernel's
 *   16-row tiles at head_dim 512 (no workgroup partials) always use SEPARATE;
 * AUTO: LAST_WG when a (slot, kv head) has at most 32 KiB of partials (one
 *   workgroup reads them all), SEPARATE otherwise.
 * Every mode gives the same results, bit for bit, when a (slot, kv head) has
 * at most 16 partial workgroups; beyond that the merge order differs. */
#define KVRT_MERGE_AUTO 0
#define KVRT_MERGE_SEPARATE 1
#define KVRT_MERGE_LAST_WG 2

/* Optional caller-owned storage for one layer (kvrt_create_with_storage).
 * Sizes must equal kvrt_layer_storage_bytes for that layer. */
typedef struct kvrt_storage {
    void *k;
    void *v;
    void *k_scale; /* INT8 only: fp32 [pool_pages, kv_heads, block] */
    void *v_scale;
} kvrt_storage;

typedef struct kvrt_counters {
    uint64_t launches;
    uint64_t appended_rows;     /* token rows appended (sum over slots, layers) */
    uint64_t appended_bytes;    /* K+V payload bytes written by append          */
    uint64_t attended_keys;     /* visible keys read by attention (per kv head) */
    uint64_t attended_bytes;    /* K+V bytes read by attention                  */
    uint64_t gathered_bytes;    /* bytes written by gather (incl. padding)      */
    uint64_t truncations;
    uint64_t truncated_rows;
    uint64_t pages_in_use;
    uint64_t pages_evicted;
    uint64_t mfma_decodes;      /* decode launches on the MFMA kernel (the rest on VALU) */
} kvrt_counters;

typedef struct kvrt_ctx kvrt_ctx;

/* ---- version / capabilities ---------------------------------------------- */
/* Replaces gemma4_listener_batch_api_version / _capabilities
 * (native/gemma4_listener_microbatch/gemma4_listener_microbatch.h:204-205;
 * probed from Python at duplex_kernel/native_listener_microbatch.py:44-59). */
uint32_t kvrt_abi_version(void);
uint64_t kvrt_capabilities(void);
const char *kvrt_strerror(int code);

/* ---- lifetime -------------------------------------------------------------- */
/* Replaces gemma4_cache_create (native/gemma4_listener_microbatch/
 * gemma4_listener_cache.cu:68-179) and the talker KV arena allocation in
 * qwen_talker_create (native/qwen_talker/qwen_talker.cu:27-113).
 * Storage is zero-initialised once at create. */
int kvrt_create(const kvrt_config *config, const kvrt_layer_spec *layers, kvrt_ctx **out);
/* Same, with caller-owned storage for every non-shared layer (entries of
 * shared layers are ignored). The caller keeps the storage alive until
 * kvrt_destroy. */
int kvrt_create_with_storage(const kvrt_config *config, const kvrt_layer_spec *layers,
                             const kvrt_storage *storage, kvrt_ctx **out);
/* Bytes of the K (== V) tensor and of the K (== V) scale tensor of a layer. */
int kvrt_layer_storage_bytes(const kvrt_config *config, const kvrt_layer_spec *layer,
                             uint64_t *kv_bytes, uint64_t *scale_bytes);
/* Replaces gemma4_cache_destroy (gemma4_listener_cache.cu:463-475). */
int kvrt_destroy(kvrt_ctx *ctx);
/* Bind the stream every later call of the context enqueues on. Binding the
 * bound stream again is a no-op. Binding a different stream returns
 * KVRT_ESTATE (nothing changes) while work the context enqueued may still be
 * running: kvrt_health or kvrt_sync_lengths synchronise the bound stream and
 * then allow the switch. A context's split-K workspace and arrival counters
 * are shared by its calls, so two streams in flight on one context would
 * race on them.
 * Replaces the bound-stream contract of the batch API
 * (gemma4_listener_microbatch_impl.inc:445-473: a second stream is refused
 * with -6; gemma4_listener.cu:2053). */
int kvrt_bind_stream(kvrt_ctx *ctx, void *hip_stream);
/* Grow the context to n_slots slots (no-op when it already has as many):
 * every slot-major layer (CONTIG / RING) moves to storage for n_slots slots,
 * the existing slots' rows, lengths, pages, masks and generations unchanged
 * and the new slots empty (zero rows, new generations); PAGED pools keep
 * their pages. A context created with kvrt_create allocates the new storage
 * itself (storage = NULL); one created with kvrt_create_with_storage passes
 * it (storage[l] for every layer l, sized by kvrt_layer_storage_bytes at the
 * new slot count; PAGED and shared entries ignored) and may free its old
 * storage once this returns. Synchronous: waits for the bound stream first.
 * KVRT_ESTATE inside a stream capture; graphs captured before the call use
 * the old buffers and must be captured again.
 * Replaces gemma4_listener_batch_ensure_capacity (bound at
 * duplex_kernel/native_listener_microbatch.py:1217-1268). */
int kvrt_grow_slots(kvrt_ctx *ctx, int32_t n_slots, const kvrt_storage *storage);
/* Device pointers of a layer's storage (shared layers report their source). */
int kvrt_layer_storage(kvrt_ctx *ctx, int32_t layer, kvrt_storage *out);

/* ---- KV operations --------------------------------------------------------- */
/* Import a prefix: k, v are [1, kv_heads, S, D] (HF DynamicCache layer view,
 * strided allowed, last dim contiguous) bf16. Sets the (slot, layer) length
 * to S. RING keeps the last ring_rows rows; PAGED allocates pages (pages
 * wholly below first_pos are not stored: first_pos = 0 stores all); INT8
 * quantises on import.
 * An import starts a session: it fails with KVRT_ESTATE, changing nothing,
 * when the (slot, layer) holds rows, when the slot has a prefix-attention
 * mask, or while the host lengths are unverified (work of this context was
 * captured into a graph since the last kvrt_sync_lengths). Reset, release
 * (truncate to 0 with the mask cleared) or a fresh slot take one. A
 * successful import renews the slot's generation: holders of the previous
 * one are refused by truncate, copy and rollover (as
 * gemma4_listener_batch_import_cache_async refuses a primed slot and takes
 * the row's identity, gemma4_listener_microbatch_impl.inc:2595, :2629-2637).
 * Replaces gemma4_cache_import_async (gemma4_listener_cache.cu:278-301),
 * qwen_talker import_cache_prefix (qwen_talker_kernels.cu:276-294,
 * qwen_talker.cu:1060-1110) and the Python copy at
 * duplex_kernel/native_qwen_talker.py:781-874. */
int kvrt_import_async(kvrt_ctx *ctx, int32_t slot, int32_t layer, const kvrt_tensor *k,
                      const kvrt_tensor *v, int32_t first_pos);

/* Append Q rows to n slots of one layer at each slot's current length:
 * k, v are [n, kv_heads, Q, D] bf16 (HF key_states layout with batch = n).
 * Lengths advance by Q. INT8 layers quantise in-kernel
 * (scale = amax/127, q = clamp(rne(x/scale), -127, 127)).
 * Replaces HF DynamicLayer.update (transformers cache_utils.py:127-146) as
 * called through duplex_kernel/kv_cache.py:95-97, gemma4_cache_append_async
 * (gemma4_listener_cache.cu:182-215) and write_audio_kv / write_joint_kv
 * (qwen_talker_kernels.cu:207-251). */
int kvrt_append_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                      const kvrt_tensor *k, const kvrt_tensor *v);

/* Write Q rows to n slots of one CONTIG bf16 layer at explicit absolute
 * positions: k, v are [n, kv_heads, Q, D]; positions is a HOST int32 array
 * [n * Q] (row r of item i lands at positions[i * Q + r]; n * Q <= 128, no
 * position twice within an item). Each (slot, layer) length becomes
 * max(length, largest position + 1); positions never written read as the
 * zeros of kvrt_create / kvrt_reset_slot_async. A position outside
 * [0, capacity) fails with KVRT_ESTATE before anything is written; Q = 0
 * changes nothing.
 * Replaces _SlotKVCache.update (duplex_kernel/future_prefix.py:523-571:
 * index_copy_ at cache_position, per-layer length = max position + 1) and
 * write_joint_kv_kernel (native/qwen_talker/qwen_talker_kernels.cu:207-225:
 * prefix row and audio row at two positions). */
int kvrt_write_positions_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                               const int32_t *positions, const kvrt_tensor *k, const kvrt_tensor *v);

/* Zero every stored row of a slot (all layers), set its lengths to 0,
 * release its pages (PAGED layers), clear its prefix-attention mask and give
 * it a new generation (the start of a session in the slot). Replaces
 * _SlotKVCache.reset (duplex_kernel/future_prefix.py:582-586) and the arena
 * memset before a talker prefix import (native/qwen_talker/
 * qwen_talker.cu:1060-1110). */
int kvrt_reset_slot_async(kvrt_ctx *ctx, int32_t slot);

/* Per-slot prefix-attention mask: key position k < P is visible only where
 * mask[k] != 0; positions >= P are unaffected. Applies on every layer of the
 * slot, on top of causal and window visibility, in kvrt_attend_decode_async,
 * kvrt_append_attend_async and kvrt_attend_prefill_async. mask is a DEVICE
 * tensor [1, P] or [P] of KVRT_INT64 (the reference's dtype), KVRT_INT32 or
 * KVRT_BOOL, 0 <= P <= KVRT_MAX_PREFIX_MASK; NULL or P = 0 clears the mask.
 * It is read on the bound stream, so the caller keeps it alive until the
 * call's work has run. Clones and copies carry the mask; kvrt_truncate
 * refuses lengths below P; kvrt_rollover_async keeps positions
 * below its prefix_len, which must be >= P. A captured HIP graph reads the
 * masks of its slots at replay time, but only if its slots had a mask when
 * it was captured.
 * Replaces the prefix_attention argument of
 * gemma4_listener_batch_import_cache_async
 * (native/gemma4_listener_microbatch/gemma4_listener_microbatch_impl.inc:
 * 2590-2621; bound at duplex_kernel/native_listener_microbatch.py:1340-1414)
 * and its use in every listener attention path (prefix_valid in
 * gemma4_listener_kernels.cuh:517-518, :595-597, :743-745,
 * gemma4_listener_attention_ordered.cu:96-101, impl.inc:2659-2660); the
 * canonical default mask (34 positions, only 0 and 33 visible) is
 * kernel_set_canonical_prefix_mask (gemma4_listener_kernels.cuh:111-118). */
int kvrt_set_prefix_attention_async(kvrt_ctx *ctx, int32_t slot, const kvrt_tensor *mask);

/* Identity and state of one slot. generation is renewed by
 * kvrt_reset_slot_async and by a clone / copy into the slot (never 0);
 * prefix_len is the length of its prefix-attention mask (0: none); min_len /
 * max_len the smallest / largest length over its non-shared layers.
 * Replaces the slot record of the batch API (session_generation,
 * prefix_len, current_position: gemma4_listener_microbatch_impl.inc:8-21)
 * and gemma4_listener_batch_get_session_state (:3920-3950). */
typedef struct kvrt_slot_info {
    uint64_t generation;
    int32_t prefix_len;
    int32_t min_len;
    int32_t max_len;
    int32_t reserved;
} kvrt_slot_info;
int kvrt_slot_info_get(kvrt_ctx *ctx, int32_t slot, kvrt_slot_info *out);

/* Gather n slots of one layer into a zero-padded batch:
 * out_k, out_v [n, kv_heads, Lmax, D] (bf16 for bf16 layers, fp32
 * dequantised for INT8 layers); row j of item i holds position
 * start_i + j for j < L_i - start_i, zeros after. mask [n, Lmax] (KVRT_BOOL:
 * 1 valid / 0 pad, or KVRT_FP32 / KVRT_BF16: 0 valid / finfo.min pad) may be
 * NULL. start_pos may be NULL (contig: 0, paged: the first live page, ring:
 * max(0, L-(W-1)) which is the HF DynamicSlidingWindowLayer retained range;
 * for contig and ring the kernel takes L from the device length, so a
 * captured call replays with the window moving along).
 * Replaces _StaticPaddingWorkspace.padded / padded_mask
 * (duplex_kernel/shape_stable_listener.py:28-69). */
int kvrt_gather_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                      const int32_t *start_pos, const kvrt_tensor *out_k,
                      const kvrt_tensor *out_v, const kvrt_tensor *mask);

/* Append k, v ([n, kv_heads, Q, D] bf16) to n slots of one layer, then gather
 * them: the same cache rows, lengths, out_k / out_v / mask and start_pos
 * rules as kvrt_append_async followed by kvrt_gather_async. For bf16
 * CONTIG / RING layers that own their rows, with Q <= max_q and contiguous
 * k / v, both happen in one launch: the new rows are taken from k / v for
 * the batch, written to the cache, and the device lengths advanced by the
 * launch's last workgroup per slot, so a captured graph replays it at
 * advancing lengths; a refused call there changes nothing. Other layers
 * take the two launches, with the two calls' effect: an append that
 * succeeds stays done if the gather is then refused.
 * Replaces the listener step's DynamicLayer.update (torch.cat,
 * duplex_kernel/kv_cache.py:95-97) followed by _StaticPaddingWorkspace.padded
 * / padded_mask (duplex_kernel/shape_stable_listener.py:28-69). */
int kvrt_append_gather_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                             const kvrt_tensor *k, const kvrt_tensor *v, const int32_t *start_pos,
                             const kvrt_tensor *out_k, const kvrt_tensor *out_v,
                             const kvrt_tensor *mask);

/* Turn-local rollback: set the length of (slot, layer) to new_len
 * (layer = -1: every layer). Moves no KV bytes. Fails with KVRT_ESTATE when
 * the slot's generation is not expected_generation (KVRT_ANY_GENERATION
 * skips the check), when expected_len >= 0 and a targeted layer's length is
 * not expected_len (the caller's position is not the slot's; -1 skips the
 * check), when new_len exceeds the current length or lies below the slot's
 * prefix-attention mask (the rewind floor), while the host lengths are
 * unverified (work of this context was captured into a graph since the
 * last kvrt_sync_lengths), or when the keys the next query (position
 * new_len) sees are no longer stored: a RING layer keeps positions from
 * (its longest length since the slot was last empty) - ring_rows on, a
 * rollback leaving that floor in place; a PAGED layer with a window keeps
 * the pages kvrt_evict did not release (without a window, new_len may not
 * fall below them). new_len == 0 (a release) is always possible; a RING
 * layer's floor then restarts at 0, and a slot's released pages are
 * forgotten once all its PAGED layers are empty. Nothing changes when it
 * fails. The device applies the edit only where it still holds the
 * lengths the host validated against; where a graph replay has advanced
 * them since (replays after a kvrt_sync_lengths), the edit is dropped whole
 * and kvrt_health reports KVRT_EFAULT (kvrt_sync_lengths then reloads the
 * device's lengths).
 * Replaces TurnKVState.truncate_to_prefix / _slice_kv
 * (duplex_kernel/kv_cache.py:99-104, :205-216), gemma4_cache_truncate_async
 * (gemma4_listener_cache.cu:409-421) and the identity-checked
 * gemma4_listener_batch_rewind_session_async
 * (gemma4_listener_microbatch_impl.inc:3588-3618: a stale identity, a
 * sequence position that is not the slot's, current_position !=
 * valid_kv_len, or a target below prefix_len -> -2). */
int kvrt_truncate(kvrt_ctx *ctx, int32_t slot, int32_t layer, int32_t new_len, uint64_t expected_generation,
                  int32_t expected_len);

/* PAGED: map the pages of the next `positions` positions of slot (after its
 * longest PAGED layer's length) now, so that appends up to there take no
 * page-table edit: a captured HIP graph of fused appends then replays across
 * page boundaries (a replay that outruns the reservation raises the device
 * flag: kvrt_health reports KVRT_EFAULT). KVRT_ENOMEM when the pool runs out
 * (nothing mapped), KVRT_ESTATE past capacity or while the host lengths are
 * unverified (captured work not yet read back). A truncate releases pages
 * wholly beyond the remaining rows, reserved ones included. No counterpart in
 * the reference (paged KV is absent there). */
int kvrt_reserve_async(kvrt_ctx *ctx, int32_t slot, int32_t positions);

/* PAGED: release every page of slot wholly below position keep_from (all
 * layers share one page table per slot). Positions below keep_from must not
 * be attended afterwards (the layer window guarantees it). No counterpart in
 * the reference (paged KV is absent there); bounded-memory decode. */
int kvrt_evict(kvrt_ctx *ctx, int32_t slot, int32_t keep_from);

/* Copy the first n_tokens positions of every non-shared layer from src_slot
 * to dst_slot in one launch (dst lengths become n_tokens), with src_slot's
 * prefix-attention mask; dst_slot gets a new generation. CONTIG layers copy
 * all n_tokens rows; RING layers the rows still in the ring; PAGED layers
 * (bf16 or int8 with scales) the rows on live pages, into freshly mapped
 * pages of dst_slot (its previous pages are released first). KVRT_ESTATE if
 * src_slot's generation is not src_generation (KVRT_ANY_GENERATION skips
 * the check), if n_tokens lies below src_slot's prefix mask, or if a key the
 * next query would see is no longer resident in src_slot; KVRT_ENOMEM
 * (nothing changed) if the pool cannot hold the copy.
 * Replaces copy_static_cache_prefix (duplex_kernel/thinker_cache.py:83-190),
 * gemma4_cache_copy_async (gemma4_listener_cache.cu:306-345) and the KV part
 * of gemma4_listener_batch_clone_session_slot_async
 * (gemma4_listener_microbatch_impl.inc:4046-4119). */
int kvrt_copy_prefix_async(kvrt_ctx *ctx, int32_t src_slot, int32_t dst_slot, int32_t n_tokens,
                           uint64_t src_generation);

/* The same copy between two contexts of identical topology (layer specs,
 * aliasing, block size, device), enqueued on dst's stream; work on src's
 * stream that produced the rows must be ordered before it by the caller.
 * Replaces the KV part of gemma4_listener_batch_copy_session_cache_async
 * (gemma4_listener_microbatch_impl.inc:4121-4172). */
int kvrt_copy_session_async(kvrt_ctx *dst, int32_t dst_slot, kvrt_ctx *src, int32_t src_slot,
                            int32_t n_tokens, uint64_t src_generation);

/* RoPE table of one non-shared bf16 layer for kvrt_rollover_async:
 * inv_freq[head_dim / 2] (host, fp32; 0 leaves a pair unrotated) and the
 * cos/sin scaling; inv_freq = NULL with n_freq = 0 removes the table.
 * Synchronous: waits for the bound stream, then uploads.
 * Replaces the d_inv_freq_sliding / d_inv_freq_full tables of the listener
 * (native/gemma4_listener_microbatch/gemma4_listener.cu:1840-1880). */
int kvrt_set_layer_rope(kvrt_ctx *ctx, int32_t layer, const float *inv_freq, int32_t n_freq, float scaling);

/* Rollover of one slot: every non-shared layer keeps positions
 * [0, prefix_len) and moves its newest retained_rows rows, positions
 * [L - retained_rows, L), to [prefix_len, prefix_len + retained_rows) (one
 * launch, overlapping ranges allowed); keys of layers with a RoPE table are
 * rotated by delta = prefix_len - (L - retained_rows) positions:
 *   c = bf16(cos(f) * scaling), s = bf16(sin(f) * scaling), f = fp32(delta * inv_freq[i]),
 *   x1' = bf16(bf16(x1 c) - bf16(x2 s)), x2' = bf16(bf16(x2 c) + bf16(x1 s))
 * for the pair (x1, x2) = (dim i, dim i + D/2). Lengths become prefix_len +
 * retained_rows. Requires CONTIG or PAGED bf16 layers (a RING drops the prefix
 * rows the next window needs), equal lengths L over the slot's layers,
 * L > prefix_len + retained_rows, 0 < retained_rows <= KVRT_MAX_ROLLOVER_ROWS,
 * prefix_len >= the slot's prefix-attention mask (which stays as it is),
 * the slot's generation equal to expected_generation (KVRT_ANY_GENERATION
 * skips the check) and, for PAGED, no evicted page.
 * Replaces gemma4_cache_rebase_async (native/gemma4_listener/
 * gemma4_listener_cache.cu:303-351) and the per-layer kernel_rope_rebase_bf16
 * launches of gemma4_listener_batch_rollover_async
 * (gemma4_listener_microbatch_impl.inc:3835-3895). */
int kvrt_rollover_async(kvrt_ctx *ctx, int32_t slot, int32_t prefix_len, int32_t retained_rows,
                        uint64_t expected_generation);

/* GQA decode attention over the last Q positions of n slots of one layer:
 * q [n, Hq, Q, D] bf16 contiguous, out [n, Hq, Q, D] bf16 contiguous.
 * q head h reads kv head h / (Hq / kv_heads) (HF repeat_kv order). Query row
 * i sits at position p = L - Q + i and sees keys k with k <= p and, for a
 * sliding layer, k >= p - W + 1. Scores s = (q.k) * scale, softmax and all
 * accumulation in fp32; out rounded to bf16 (RNE). (Hq / kv_heads) * Q must
 * be <= 16, and <= 8 for INT8 layers.
 * Replaces HF sdpa_attention_forward over repeat_kv'd K/V
 * (shape_stable_listener.py:241-251), gemma4_listener_debug_attention
 * (gemma4_listener_aten.cpp:100-286), kernel_stream_sdpa_q4_bf16
 * (gemma4_listener_kernels.cuh:534-665) and qwen_attention_gqa
 * (qwen_talker_kernels.cu:875-921). */
int kvrt_attend_decode_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                             const kvrt_tensor *q, const kvrt_tensor *out, float scale);

/* Fused per-layer decode step: append k, v ([n, kv_heads, Q, D]) then attend
 * q ([n, Hq, Q, D]) — the same results as kvrt_append_async followed by
 * kvrt_attend_decode_async, in fewer launches. Replaces the per-session
 * append + attention pair of gemma4_batch_execute_layer
 * (gemma4_listener_microbatch_impl.inc:2939-2962) and the talker
 * write_audio_kv + repeat_kv + SDPA sequence (qwen_talker.cu:693-756). */
int kvrt_append_attend_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                             const kvrt_tensor *q, const kvrt_tensor *k, const kvrt_tensor *v,
                             const kvrt_tensor *out, float scale);

/* Chunked-prefill attention on MFMA: q [n, Hq, Q, D] bf16 contiguous holds
 * the queries of the last Q positions of each slot (append the chunk's K/V
 * first, e.g. with kvrt_append_async); out likewise. Same visibility, scale
 * and GQA head map as kvrt_attend_decode_async, for any Q <= length. P
 * enters the P.V product as a sum of two bf16 terms (~2^-17 relative);
 * scores, softmax and both products accumulate in fp32. bf16 layers only;
 * any Hq / kv_heads. RING layers need ring_rows >= Q + window - 1, PAGED
 * layers the pages of the oldest visible key (KVRT_ESTATE otherwise).
 * Replaces kernel_prefill_sdpa_bf16 (native/gemma4_listener_microbatch/
 * gemma4_listener_kernels.cuh:692-790) and the Q3..Q8 text-append attention
 * of the listener batch API (gemma4_listener_microbatch_impl.inc:3476-3586). */
int kvrt_attend_prefill_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                              const kvrt_tensor *q, const kvrt_tensor *out, float scale);

/* Talker visibility of one slot for kvrt_attend_talker_async. Positions are
 * absolute cache rows: [0, prefix_start) is the stable text, [prefix_start,
 * audio_start) the reserved prefix frames of which [prefix_start,
 * prefix_position] are visible, [audio_start, audio_position] the audio
 * frames so far. prefix_attention_mode: 0 audio queries see the visible
 * prefix, 1 they do not, 2 they see it with prefix_log_gate -
 * log(visible_prefix_count) (rounded to bf16) added to those scores. */
typedef struct kvrt_talker_mask {
    int32_t prefix_start;
    int32_t audio_start;
    int32_t prefix_position;
    int32_t audio_position;
    int32_t prefix_attention_mode;
    int32_t visible_prefix_count;
    float prefix_log_gate;
} kvrt_talker_mask;

/* Talker attention for n slots of one CONTIG bf16 layer with window 0:
 * q, out [n, Hq, Q, D] bf16 contiguous with Q = 2 (JOINT step: row 0 the
 * prefix query at prefix_position, row 1 the audio query at audio_position)
 * or Q = 1 (audio-only query at audio_position, prefix_position being the
 * last visible prefix frame). Key k is visible to
 *   the prefix query: k < prefix_start or prefix_start <= k <= prefix_position
 *   an audio query:   k < prefix_start, prefix_start <= k <= prefix_position
 *                     unless mode 1, or audio_start <= k <= audio_position
 * masks[i] describes slot i; write the step's K/V rows first (e.g. with
 * kvrt_write_positions_async). Requires 0 <= prefix_start <= prefix_position
 * < audio_start <= audio_position < length(slot, layer), mode <= 2, a finite
 * gate and visible_prefix_count > 0 in mode 2 (KVRT_EINVAL / KVRT_ESTATE
 * otherwise). Scores, softmax and accumulation in fp32, out bf16 (RNE).
 * Replaces build_joint_mask_kernel / build_audio_only_mask_kernel and their
 * launchers (native/qwen_talker/qwen_talker_kernels.cu:296-347, :759-807)
 * with the repeat_kv + masked SDPA they feed (qwen_talker.cu:718-756,
 * qwen_talker_aten_attention.cpp:150-160). */
int kvrt_attend_talker_async(kvrt_ctx *ctx, int32_t layer, int32_t n, const int32_t *slots,
                             const kvrt_tensor *q, const kvrt_tensor *out, float scale,
                             const kvrt_talker_mask *masks);

/* ---- context-free tensor kernels ------------------------------------------ */
/* Decode attention over caller-owned HF-shaped K/V: k, v [n, kv_heads, Lmax, D]
 * bf16 (strided, last dim contiguous), lengths int32[n] in DEVICE memory,
 * q/out [n, Hq, Q, D]; window as above (0 = global); row j of item b is key
 * position j. prefix_attention (may be NULL) is a DEVICE tensor [n, P] of
 * KVRT_INT64 / KVRT_INT32 / KVRT_BOOL, P <= KVRT_MAX_PREFIX_MASK: key j < P
 * of item b is visible only where prefix_attention[b, j] != 0. Used for the
 * padded batch produced by kvrt_gather_async and for HF cache objects.
 * The split-K partials live in a workspace the library keeps per (device,
 * stream): calls on one stream share it in stream order, calls on different
 * streams never do. A call that would need a larger workspace while its
 * stream is being captured returns KVRT_ESTATE (make one eager call of the
 * largest shape first); outgrown workspaces are kept until the process ends,
 * since captured graphs may still use them. Lengths beyond Lmax are clamped
 * and raise the stream's error flag (kvrt_tensors_status).
 * Replaces sdpa_attention_forward on padded K/V + mask
 * (shape_stable_listener.py:232-251) and the listener's prefix_valid term
 * (gemma4_listener_kernels.cuh:517-518). */
int kvrt_attend_tensors_async(const kvrt_tensor *q, const kvrt_tensor *k, const kvrt_tensor *v,
                              const int32_t *device_lengths, const kvrt_tensor *prefix_attention,
                              const kvrt_tensor *out, float scale, int32_t window, void *hip_stream);

/* The same attention with no allocation: the split-K partials go to a
 * scratch array the library holds on each GPU (KVRT_NOALLOC_SCRATCH_BYTES, set
 * up on the device's first call) instead of an allocated workspace, and the
 * call makes no hipMalloc / hipFree or allocating library call. Same
 * arguments, checks and results as kvrt_attend_tensors_async, except: a call
 * whose partials would not fit uses fewer split-K workgroups (results then
 * differ from kvrt_attend_tensors_async in fp32 rounding only), and one that
 * does not fit even with one workgroup per (item, kv head) returns
 * KVRT_EINVAL; lengths beyond Lmax are clamped without a report. Every call on
 * a GPU shares that GPU's scratch: calls that overlap on one GPU (two
 * streams, or two host threads) race, so callers serialise them.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
#define KVRT_NOALLOC_SCRATCH_BYTES (16u << 20)
int kvrt_attend_tensors_noalloc_async(const kvrt_tensor *q, const kvrt_tensor *k, const kvrt_tensor *v,
                                      const int32_t *device_lengths, const kvrt_tensor *prefix_attention,
                                      const kvrt_tensor *out, float scale, int32_t window, void *hip_stream);

/* Synchronise hip_stream, then report and clear the error flag of the
 * stream's kvrt_attend_tensors_async workspace: KVRT_OK, KVRT_EFAULT (a
 * length beyond its K/V rows was clamped) or KVRT_EDEVICE. KVRT_OK when the
 * stream has no workspace yet. Replaces the talker's device error flag check
 * (native/qwen_talker/qwen_talker_kernels.cu:243-246) for this path. */
int kvrt_tensors_status(void *hip_stream);

/* Row copy between two 4-D strided tensors of the same element size
 * (2 or 4 bytes) over dims (d0, d1, rows, D): dst[:, :, :rows] = src[:, :, :rows].
 * Replaces the per-layer StaticLayer slice copy of copy_static_cache_prefix
 * (duplex_kernel/thinker_cache.py:164-170). */
int kvrt_copy_rows_async(const kvrt_tensor *src, const kvrt_tensor *dst, int64_t rows,
                         void *hip_stream);

/* ---- state / diagnostics ----------------------------------------------------- */
/* Host-authoritative length of (slot, layer). Replaces
 * gemma4_cache_valid_kv_len (gemma4_listener_cache.cu:423-425) and
 * _kv_seq_len (duplex_kernel/kv_cache.py:190-201). */
int kvrt_session_state(kvrt_ctx *ctx, int32_t slot, int32_t layer, int32_t *length);
/* Synchronise the bound stream and reload the host lengths from the device
 * mirror. Needed after replaying a captured HIP graph of append / fused
 * calls: replays advance the device lengths only. After work of the context
 * was captured, import and truncate are refused until this call. The split count and
 * workspace of a captured call are fixed at capture; lengths must stay within
 * capacity and, for PAGED layers, within mapped pages. No counterpart in the
 * reference (its graphs use a device cursor, qwen_talker_kernels.cu:349-374). */
int kvrt_sync_lengths(kvrt_ctx *ctx);
int kvrt_get_counters(kvrt_ctx *ctx, kvrt_counters *out);
/* Synchronise the bound stream, then report KVRT_OK, KVRT_EPOISONED,
 * KVRT_EDEVICE (HIP error) or KVRT_EFAULT (kernel-side bounds flag).
 * Replaces the stream-query health path (gemma4_listener.cu:180-192) and the
 * talker device error flag (qwen_talker_kernels.cu:243-246). */
int kvrt_health(kvrt_ctx *ctx);
/* Host-side fault injection for failure-path tests: the next mutating call
 * fails as a device enqueue failure (poisoning the ctx). No kernel runs. */
int kvrt_debug_inject_failure(kvrt_ctx *ctx);

#ifdef __cplusplus
}
#endif

#endif /* KVRT_H */

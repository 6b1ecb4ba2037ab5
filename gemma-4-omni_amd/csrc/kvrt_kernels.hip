// kvrt_kernels.hip — gfx950 kernels of the KV hot path.
//
//   append_kernel   per-frame K/V append / prefix import into CONTIG, RING or
//                   PAGED rows (bf16 copy or int8 quantise-on-write)
//   gather_kernel   ragged N-stream gather into a zero-padded batch + mask
//   decode_kernel   GQA split-K decode attention, one wave per key split,
//                   fp32 online softmax; the waves of a workgroup merge in
//                   LDS and write one partial (m, l, acc) per workgroup
//   merge_kernel    log-sum-exp merge of the partials in fixed order
//                   (deterministic) -> bf16, then the fused length advance
//   set_i32_kernel  length / page-table edits carried in the kernarg block
//   copy_rows_kernel, zero_kernel, slot_copy_kernel, slot_rebase_kernel
//
// Every memory-bound loop moves 16 B per lane with consecutive lanes on
// consecutive addresses (one 1 KiB transaction per wave instruction).
#include <type_traits>

#include "kvrt_device.h"
#include "kvrt_internal.h"

namespace kvrt {

constexpr float kNegBig = -1.0e30f;  // running-max start; exp2(kNegBig - m) == 0
// Lazy online softmax: a running max m (log2 units) moves only when a block's
// max exceeds it by more than kRescaleSlack, so p = 2^(s - m) stays <= 2^8
// and the accumulator rescale runs a few times per wave instead of on most
// blocks. Exact: l and the accumulator always refer to the same m, and every
// merge weights a partial by its own m.
constexpr float kRescaleSlack = 8.0f;

// Row number of position pos of a head on a PAGED page, in pool order
// ((page, head, pos % rows)); -1 if the page is unmapped or out of the pool.
// 32-bit arithmetic: the host keeps pool_pages below 2^24 and the pool's rows
// below 2^31, so page * (kv_heads * rows) is a 24-bit product.
__device__ __forceinline__ int page_row(const KVView &v, int page, int head, int pos) {
    if (page < 0 || page >= v.pool_pages) return -1;
    return (int)__umul24((unsigned)page, (unsigned)(v.kv_heads * v.rows)) + head * v.rows + (pos & (v.rows - 1));
}

// Element offset of the first element of row (slot, head, pos); -1 if the
// page is unmapped or out of the pool.
template <int LAYOUT>
__device__ __forceinline__ int64_t row_offset(const KVView &v, int slot, int head, int pos, int D) {
    if constexpr (LAYOUT == KVRT_LAYOUT_CONTIG) {
        return slot * v.slot_stride + head * v.head_stride + (int64_t)pos * v.row_stride;
    } else if constexpr (LAYOUT == KVRT_LAYOUT_RING) {
        return slot * v.slot_stride + head * v.head_stride + (int64_t)(pos % v.rows) * v.row_stride;
    } else {
        const int lp = pos >> v.block_shift;
        if (pos < 0 || lp >= v.pt_stride) return -1;
        const int page = v.page_table[(int64_t)slot * v.pt_stride + lp];
        const int row = page_row(v, page, head, pos);
        return row < 0 ? -1 : (int64_t)row * D;
    }
}

// Prefix-attention mask of a slot as a wave holds it: its length plen (0: no
// mask; wave-uniform, in an SGPR) and, in every lane, mask word (lane & 15).
// The record is read only when the launch carries masks, so launches without
// them load nothing. Both values are waited for here, so callers issue this
// next to their length load (one memory round trip for both) and before any
// LDS DMA: the compiler does not count inline-assembly DMAs, and a wait it
// placed for these loads inside a DMA-pipelined loop would drain the ring.
__device__ __forceinline__ void load_prefix(const PrefixMask *pm, int slot, int lane, int &plen, uint32_t &pw) {
    plen = 0;
    pw = 0xffffffffu;
    if (pm != nullptr) {
        plen = __builtin_amdgcn_readfirstlane(pm[slot].len);
        pw = pm[slot].bits[lane & (kPrefixWords - 1)];
        asm volatile("" ::"v"(pw));  // the word is in its register from here on
    }
}
// Mask bit of key position key (0 <= key < KVRT_MAX_PREFIX_MASK): the word
// comes from the lane that holds it (ds_bpermute), so every lane of the wave
// must call this together.
__device__ __forceinline__ bool prefix_bit(uint32_t pw, int key) {
    const uint32_t w = (uint32_t)__shfl((int)pw, (key >> 5) & (kPrefixWords - 1));
    return ((w >> (key & 31)) & 1u) != 0;
}
// Mask bits of the 8 keys k0 .. k0 + 7 (k0 >= 0; bit j: key k0 + j passes
// the mask of length plen), branch-free: the two words they span come from
// the lanes that hold them, keys at or past plen pass. Every lane of the wave
// must call this together.
__device__ __forceinline__ uint32_t prefix_bits8(uint32_t pw, int k0, int plen) {
    const int w = k0 >> 5;
    const uint32_t lo = (uint32_t)__shfl((int)pw, w & (kPrefixWords - 1));
    const uint32_t hi = (uint32_t)__shfl((int)pw, (w + 1) & (kPrefixWords - 1));
    const uint32_t bits = (uint32_t)((((uint64_t)hi << 32) | lo) >> (k0 & 31)) & 0xffu;
    const int past = plen - k0;  // keys j >= past are beyond the mask
    const uint32_t open = past <= 0 ? 0xffu : past >= 8 ? 0u : (0xffu << past) & 0xffu;
    return bits | open;
}


// Item of grid z-index z of a PAGED decode: order[] read as aligned words
// through the scalar cache (a byte read is a vector load: one more memory
// round trip ahead of the slot and length loads).
static_assert(offsetof(DecodeArgs, order) % 4 == 0 && kMaxItems % 4 == 0, "order[] in whole words");
__device__ __forceinline__ int launch_item(const DecodeArgs &a, int z) {
    uint32_t w;
    __builtin_memcpy(&w, a.order + 4 * (z >> 2), 4);
    return (int)((w >> (8 * (z & 3))) & 0xffu);
}

// q = x / d and r = x % d for x >= 0 and a wave-uniform d > 0: a shift and a
// mask when d is a power of two (a uniform branch), else the division.
__device__ __forceinline__ void udivmod_uniform(int x, int d, int &q, int &r) {
    if ((d & (d - 1)) == 0) {
        q = x >> __builtin_ctz((unsigned)d);
        r = x & (d - 1);
    } else {
        q = x / d;
        r = x - q * d;
    }
}
__device__ __forceinline__ int umod_uniform(int x, int d) {
    int q, r;
    udivmod_uniform(x, d, q, r);
    return r;
}

// A wave's window of page-table entries: lane i holds the entry of logical
// page win0 + i of the slot (-1 past the table).
__device__ __forceinline__ int load_page_window(const KVView &v, int slot, int win0, int lane) {
    const int lp = win0 + lane;
    return lp < v.pt_stride ? v.page_table[(int64_t)slot * v.pt_stride + lp] : -1;
}
// Element offset of row pos of a head on a page; -1 if the page is unmapped
// or out of the pool.
__device__ __forceinline__ int64_t page_row_offset(const KVView &v, int page, int head, int pos, int D) {
    const int row = page_row(v, page, head, pos);
    return row < 0 ? -1 : (int64_t)row * D;
}

// Symmetric int8 quantisation of one (token, head) row whose D values are
// spread over G consecutive lanes, NV per lane: scale = amax / 127,
// q = clamp(rne(x / scale), -127, 127), zeros when amax == 0. q packs this
// lane's NV values, 4 per word; returns the scale. Every lane of the G must
// call it together (the amax is reduced across them). The append kernel and
// the fused int8 decode both quantise through here, so a row appended either
// way holds the same bytes.
template <int NV, int G>
__device__ __forceinline__ float quantize_row(const float (&x)[NV], uint32_t (&q)[NV / 4]) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = group_max<G>(amax);
    const float sc = amax / 127.0f;
#pragma unroll
    for (int w = 0; w < NV / 4; ++w) q[w] = 0u;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int qi = amax > 0.f ? (int)fminf(fmaxf(rintf(x[i] / sc), -127.f), 127.f) : 0;
        q[i >> 2] |= ((uint32_t)(qi & 0xff)) << (8 * (i & 3));
    }
    return sc;
}

// quantize_row of 16 bf16 values (two 16-B words), G lanes per row.
template <int G>
__device__ __forceinline__ float quantize16_bf16(const uint4 (&src)[2], uint4 &q) {
    float f[16];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 x = src[h];
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[8 * h + 2 * i] = bf16_lo(w[i]);
            f[8 * h + 2 * i + 1] = bf16_hi(w[i]);
        }
    }
    uint32_t qw[4];
    const float sc = quantize_row<16, G>(f, qw);
    q = make_uint4(qw[0], qw[1], qw[2], qw[3]);
    return sc;
}

// Element offset of the new row (slot, head, pos) of a fused append: a PAGED
// row's page comes from the launch's page-table edits where one maps it (the
// table entry is written by the same launch), else from the table.
template <int LAYOUT>
__device__ __forceinline__ int64_t new_row_offset(const DecodeArgs &a, int slot, int head, int pos, int D) {
    if constexpr (LAYOUT == KVRT_LAYOUT_PAGED) {
        const int lp = pos >> a.kv.block_shift;
        if (pos < 0 || lp >= a.kv.pt_stride) return -1;
        const int idx = slot * a.kv.pt_stride + lp;
        int page = -2;
        for (int i = 0; i < a.n_upd; ++i) page = a.upd_idx[i] == idx ? a.upd_val[i] : page;
        if (page == -2) return row_offset<LAYOUT>(a.kv, slot, head, pos, D);
        return page_row_offset(a.kv, page, head, pos, D);
    } else {
        return row_offset<LAYOUT>(a.kv, slot, head, pos, D);
    }
}

// Fused int8 append: the launch's Qn new rows of (item, kv head) quantised
// exactly as the append kernel quantises them (D/16 lanes of 16 values per
// row, quantize16_bf16) by the calling wave into LDS (row r: 16-byte units
// nrow_k / nrow_v[r * D/16 + unit], scales nrow_s[r] (K) and nrow_s[NQ + r]
// (V)), for the decode's pass or tile that attends over them; with store,
// also into the cache with their scales (the one wave whose key range
// starts at or before the first new row does that).
template <int D, int NQ, int LAYOUT>
__device__ __forceinline__ void i8_new_rows(const DecodeArgs &a, int item, int slot, int kvh, int hkv, int len,
                                            int Qn, int lane, bool store, uint4 *nrow_k, uint4 *nrow_v,
                                            float *nrow_s) {
    constexpr int LPR = D / 16, RPW = 64 / LPR;
    const int sub = lane / LPR, seg = lane % LPR;
    const int64_t base = (((int64_t)item * hkv + kvh) * Qn) * D + seg * 16;
    for (int r0 = 0; r0 < Qn; r0 += RPW) {
        const int r = r0 + sub;
        const bool live = r < Qn;
        const int64_t on = base + (int64_t)(live ? r : 0) * D;
        uint4 kx2[2], vx2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            kx2[h] = *reinterpret_cast<const uint4 *>(a.k_new + on + 8 * h);
            vx2[h] = *reinterpret_cast<const uint4 *>(a.v_new + on + 8 * h);
        }
        uint4 kq, vq;
        const float ks = quantize16_bf16<LPR>(kx2, kq);
        const float vs = quantize16_bf16<LPR>(vx2, vq);
        if (live) {
            nrow_k[r * LPR + seg] = kq;
            nrow_v[r * LPR + seg] = vq;
            if (seg == 0) {
                nrow_s[r] = ks;
                nrow_s[NQ + r] = vs;
            }
            if (store) {
                const int64_t dst = new_row_offset<LAYOUT>(a, slot, kvh, len + r, D);
                if (dst < 0) {
                    a.err[0] = 1;
                } else {
                    *reinterpret_cast<uint4 *>(static_cast<int8_t *>(a.kv.k) + dst + seg * 16) = kq;
                    *reinterpret_cast<uint4 *>(static_cast<int8_t *>(a.kv.v) + dst + seg * 16) = vq;
                    if (seg == 0) {
                        a.kv.ks[dst / D] = ks;
                        a.kv.vs[dst / D] = vs;
                    }
                }
            }
        }
    }
}

// The launch's page-table edits (DecodeArgs::n_upd), written by its first
// workgroup.
__device__ __forceinline__ void apply_page_edits(const DecodeArgs &a) {
    if (a.n_upd > 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
        for (int i = threadIdx.x; i < a.n_upd; i += blockDim.x) a.kv.page_table[a.upd_idx[i]] = a.upd_val[i];
}

// ---------------------------------------------------------------------------
// append / import
// ---------------------------------------------------------------------------
// grid (grid_x, n_items), 256 threads. Thread chunk = 8 elements of one row.
// Mode 0 (device cursor) runs with grid_x == 1, so the workgroup that
// advances an item's length is the only one that reads it.
template <int D, int KDT, int LAYOUT>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
    constexpr int LPR = D / 8;
    const int item = blockIdx.y;
    const int slot = a.slots[item];
    if constexpr (LAYOUT == KVRT_LAYOUT_PAGED) {
        for (int i = threadIdx.x; i < a.n_upd; i += blockDim.x) {
            const int idx = a.upd_idx[i];
            if (idx / a.kv.pt_stride == slot) a.kv.page_table[idx] = a.upd_val[i];
        }
        __syncthreads();
    }
    int32_t *lp = a.len.lens + (int64_t)slot * a.len.stride + a.len.offset;
    // Both values are loaded and then selected: a select between the two
    // addresses would take the address of the kernel argument block and
    // copy it to scratch memory.
    const int dev_len = *lp;
    const int host_pos = a.base_pos;
    const int pos0 = a.import_mode == 0 ? dev_len : host_pos;
    const int64_t chunks = (int64_t)a.kv.kv_heads * a.rows * LPR;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += step) {
        const int seg = (int)(c % LPR);
        const int64_t rowid = c / LPR;
        const int r = (int)(rowid % a.rows);
        const int h = (int)(rowid / a.rows);
        const int pos = a.import_mode == 2 ? a.pos[item * a.rows + r] : pos0 + r;
        if (a.import_mode == 1 && pos < a.keep_from) continue;  // uniform over the row group
        const int64_t src = item * a.src_item_stride + h * a.src_head_stride + r * a.src_row_stride + seg * 8;
        const uint4 kx = *reinterpret_cast<const uint4 *>(a.k_src + src);
        const uint4 vx = *reinterpret_cast<const uint4 *>(a.v_src + src);
        bool ok = true;
        if constexpr (LAYOUT == KVRT_LAYOUT_CONTIG) ok = pos < a.kv.rows;
        const int64_t dst = ok ? row_offset<LAYOUT>(a.kv, slot, h, pos, D) : -1;
        if (dst < 0) {
            if (seg == 0) a.err[0] = 1;
            continue;
        }
        if constexpr (KDT == KVRT_BF16) {
            *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.kv.k) + dst + seg * 8) = kx;
            *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.kv.v) + dst + seg * 8) = vx;
        } else {
            // symmetric int8 per (token, head), D/8 lanes per row
            const uint32_t kw[4] = {kx.x, kx.y, kx.z, kx.w};
            const uint32_t vw[4] = {vx.x, vx.y, vx.z, vx.w};
            float kf[8], vf[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kf[2 * i] = bf16_lo(kw[i]);
                kf[2 * i + 1] = bf16_hi(kw[i]);
                vf[2 * i] = bf16_lo(vw[i]);
                vf[2 * i + 1] = bf16_hi(vw[i]);
            }
            uint32_t kq[2], vq[2];
            const float ksc = quantize_row<8, LPR>(kf, kq);
            const float vsc = quantize_row<8, LPR>(vf, vq);
            *reinterpret_cast<uint2 *>(static_cast<int8_t *>(a.kv.k) + dst + seg * 8) = make_uint2(kq[0], kq[1]);
            *reinterpret_cast<uint2 *>(static_cast<int8_t *>(a.kv.v) + dst + seg * 8) = make_uint2(vq[0], vq[1]);
            if (seg == 0) {
                a.kv.ks[dst / D] = ksc;
                a.kv.vs[dst / D] = vsc;
            }
        }
    }
    __syncthreads();
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (a.import_mode == 2) *lp = max(*lp, a.pos_end[item]);
        else *lp = pos0 + a.rows;
    }
}

// ---------------------------------------------------------------------------
// gather
// ---------------------------------------------------------------------------
// grid (ceil(lmax / GatherRows<D>), kv_heads, n_items), 256 threads. A
// workgroup copies GatherRows<D> padded rows of one (item, head): LPR = D/8
// lanes per row (8 elements = 16 B each), kGatherUnroll rows per thread, all
// of whose loads are issued before the first store. Rows past the item's
// valid length are written as zeros; head 0's workgroups also write the mask
// entries of their rows. (A flat grid-stride loop over 16-B chunks spent two
// 64-bit divisions per chunk on the row and head.)
// Fused append (a.k_new set; bf16 CONTIG / RING): the item's device length L0
// is the append position; rows L0 .. L0 + qn - 1 of the gathered range come
// from k_new / v_new, workgroup x = 0 of each (item, head) also stores them
// into the cache (no workgroup of the launch reads those cache rows; RING rows
// overwritten hold positions before every gathered start, which ring_rows >=
// window + max_q - 1 guarantees), and the last workgroup of the item to
// arrive (counted per (item, head), then per item) advances its length by
// qn, after every workgroup has read L0.
constexpr int kGatherUnroll = 4;
template <int D>
constexpr int gather_rows() { return 256 / (D / 8) * kGatherUnroll; }
template <int D, int KDT, int LAYOUT>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
    constexpr int LPR = D / 8;
    constexpr int RPP = 256 / LPR;  // rows per pass of the workgroup
    constexpr int U = kGatherUnroll;
    constexpr bool FUSE = KDT == KVRT_BF16 && LAYOUT != KVRT_LAYOUT_PAGED;
    const int item = blockIdx.z;
    const int h = blockIdx.y;
    const int slot = a.slots[item];
    const int L0 = a.len.lens[(int64_t)slot * a.len.stride + a.len.offset];
    const bool fused = FUSE && a.k_new != nullptr;
    const int Qn = fused ? a.qn : 0;
    const int L = L0 + Qn;
    // appended row r of this (item, head), 16 B at column chunk sg
    auto new_row = [&](const uint16_t *src, int r, int sg) __attribute__((always_inline)) {
        return *reinterpret_cast<const uint4 *>(src + (((int64_t)item * gridDim.y + h) * Qn + r) * D + sg * 8);
    };
    if (fused && blockIdx.x == 0) {
        for (int c = threadIdx.x; c < Qn * (D / 8); c += blockDim.x) {
            const int r = c / (D / 8), sg = c % (D / 8);
            const int pos = L0 + r;
            const int64_t dst = (LAYOUT == KVRT_LAYOUT_CONTIG && pos >= a.kv.rows)
                                    ? -1 : row_offset<LAYOUT>(a.kv, slot, h, pos, D);
            if (dst < 0) {
                a.err[0] = 1;
                continue;
            }
            const uint4 kx = new_row(a.k_new, r, sg), vx = new_row(a.v_new, r, sg);
            store_agent16(static_cast<uint16_t *>(a.kv.k) + dst + sg * 8, kx);
            store_agent16(static_cast<uint16_t *>(a.kv.v) + dst + sg * 8, vx);
        }
    }
    int start;
    if (a.has_start) start = a.start[item];
    else if (LAYOUT == KVRT_LAYOUT_RING && a.window > 0) start = max(0, L - (a.window - 1));
    else start = 0;
    const int valid = max(0, L - start);
    const int seg = threadIdx.x % LPR;
    const int j0 = blockIdx.x * (RPP * U) + threadIdx.x / LPR;
    float kf[U][8], vf[U][8];
    uint4 kx[U], vx[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        kx[u] = vx[u] = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) kf[u][i] = vf[u][i] = 0.f;
        const int j = j0 + u * RPP;
        if (fused && j < valid && j < a.lmax && start + j >= L0) {
            kx[u] = new_row(a.k_new, start + j - L0, seg);
            vx[u] = new_row(a.v_new, start + j - L0, seg);
        } else if (j < valid && j < a.lmax) {
            int64_t src = row_offset<LAYOUT>(a.kv, slot, h, start + j, D);
            if (LAYOUT == KVRT_LAYOUT_CONTIG && start + j >= a.kv.rows) src = -1;
            if (src < 0) {
                if (seg == 0) a.err[0] = 1;
            } else if constexpr (KDT == KVRT_BF16) {
                kx[u] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.kv.k) + src + seg * 8);
                vx[u] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.kv.v) + src + seg * 8);
            } else {
                const uint2 kq = *reinterpret_cast<const uint2 *>(static_cast<const int8_t *>(a.kv.k) + src + seg * 8);
                const uint2 vq = *reinterpret_cast<const uint2 *>(static_cast<const int8_t *>(a.kv.v) + src + seg * 8);
                const float ks = a.kv.ks[src / D], vs = a.kv.vs[src / D];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t kw = i < 4 ? kq.x : kq.y, vw = i < 4 ? vq.x : vq.y;
                    kf[u][i] = (float)(int8_t)(kw >> (8 * (i & 3))) * ks;
                    vf[u][i] = (float)(int8_t)(vw >> (8 * (i & 3))) * vs;
                }
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int j = j0 + u * RPP;
        if (j >= a.lmax) continue;
        const int64_t o = item * a.out_item_stride + h * a.out_head_stride + j * a.out_row_stride + seg * 8;
        if (a.out_fp32) {
            if constexpr (KDT == KVRT_BF16) {
                const uint32_t kw[4] = {kx[u].x, kx[u].y, kx[u].z, kx[u].w};
                const uint32_t vw[4] = {vx[u].x, vx[u].y, vx[u].z, vx[u].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    kf[u][2 * i] = bf16_lo(kw[i]); kf[u][2 * i + 1] = bf16_hi(kw[i]);
                    vf[u][2 * i] = bf16_lo(vw[i]); vf[u][2 * i + 1] = bf16_hi(vw[i]);
                }
            }
            float4 *ko = reinterpret_cast<float4 *>(static_cast<float *>(a.out_k) + o);
            float4 *vo = reinterpret_cast<float4 *>(static_cast<float *>(a.out_v) + o);
            ko[0] = make_float4(kf[u][0], kf[u][1], kf[u][2], kf[u][3]);
            ko[1] = make_float4(kf[u][4], kf[u][5], kf[u][6], kf[u][7]);
            vo[0] = make_float4(vf[u][0], vf[u][1], vf[u][2], vf[u][3]);
            vo[1] = make_float4(vf[u][4], vf[u][5], vf[u][6], vf[u][7]);
        } else {
            *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.out_k) + o) = kx[u];
            *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.out_v) + o) = vx[u];
        }
    }
    if (a.mask != nullptr && h == 0 && threadIdx.x < RPP * U) {
        const int j = blockIdx.x * (RPP * U) + threadIdx.x;
        if (j < a.lmax) {
            const bool ok = j < valid;
            const int64_t mo = item * a.mask_item_stride + j;
            if (a.mask_dtype == KVRT_BOOL) static_cast<uint8_t *>(a.mask)[mo] = ok ? 1 : 0;
            else if (a.mask_dtype == KVRT_FP32) static_cast<float *>(a.mask)[mo] = ok ? 0.f : -3.4028234663852886e38f;
            else static_cast<uint16_t *>(a.mask)[mo] = ok ? (uint16_t)0 : (uint16_t)0xff7f;  // bf16 finfo.min
        }
    }
    if (fused) {
        __syncthreads();  // every thread of the workgroup has used L0
        if (threadIdx.x == 0) {
            uint32_t *hc = a.cnt + kCntGatherHead(item, h);
            if (arrive_agent(hc) == gridDim.x - 1) {  // the last of the (item, head)
                clear_agent(hc);
                uint32_t *ic = a.cnt + kCntGatherItem(item);
                if (arrive_agent(ic) == gridDim.y - 1) {  // the last head of the item
                    clear_agent(ic);
                    a.len.lens[(int64_t)slot * a.len.stride + a.len.offset] = L;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// decode attention (split-K)
// ---------------------------------------------------------------------------
// LDS DMA: global_load_lds_dwordx4 moves lane l's 16 bytes at g to LDS byte
// M0 + 16 * l without passing through registers. It is issued from inline
// assembly (the LDS address is an M0 operand the compiler sets up), so the
// compiler neither tracks these loads nor inserts its own (all-or-nothing)
// waits for them: the decode waits with explicit vmcnt waits — vector loads
// complete in issue order, so vmcnt(N) means every DMA but the N most recent
// has landed — and reads the LDS back only after such a wait.
__device__ __forceinline__ void dma_load16(const void *g, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds) : "memory");
}
// 4 bytes per lane, to LDS byte M0 + 4 * l.
__device__ __forceinline__ void dma_load4(const void *g, uint32_t lds) {
    asm volatile("global_load_lds_dword %0, off nt" ::"v"(g), "{m0}"(lds) : "memory");
}
// The same without the streaming hint, for tiles other workgroups read again.
__device__ __forceinline__ void dma_load16_cached(const void *g, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmem() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most n * STEP vector memory operations are outstanding,
// n in [0, NMAX] (wave-uniform).
template <int STEP, int NMAX>
__device__ __forceinline__ void wait_vmem_steps(int n) {
    if constexpr (NMAX > 0) {
        if (n >= NMAX) {
            wait_vmem<NMAX * STEP>();
            return;
        }
        wait_vmem_steps<STEP, NMAX - 1>(n);
    } else {
        wait_vmem<0>();
    }
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <class T>
__device__ __forceinline__ uint32_t lds_addr(const T *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T *)p;
}

// LDS floats a decode workgroup needs for its cross-wave merge: the partials
// of waves 1..3, when R * D is small enough to stage them.
// Online merge of the partials sp = j, j + G, ... < n of one output element
// into (M, L, O), 16 at a time; ld(sp, ml, acc) reads partial sp. The merge
// kernel and the single-launch decode tail both use it, so the two paths
// round identically.
template <int G, class Ld>
__device__ __forceinline__ void merge_partials(int j, int n, Ld ld, float &M, float &L, float &O) {
    constexpr int B = 16;
    for (int s0 = j; s0 < n; s0 += B * G) {
        float2 m[B];
        float v[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int sp = s0 + u * G;
            m[u] = make_float2(kNegBig, 0.f);
            v[u] = 0.f;
            if (sp < n) ld(sp, m[u], v[u]);
        }
        float bm = M;
#pragma unroll
        for (int u = 0; u < B; ++u) bm = fmaxf(bm, m[u].x);
        const float c = __builtin_amdgcn_exp2f(M - bm);
        L *= c;
        O *= c;
        M = bm;
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const float w = __builtin_amdgcn_exp2f(m[u].x - M);
            L = fmaf(m[u].y, w, L);
            O = fmaf(v[u], w, O);
        }
    }
}

// Single-launch decode: after every workgroup has stored its partials (with
// store_agent), the last workgroup of each (item, kv head) to arrive merges
// them in the merge kernel's order and writes the output; the last of an
// item's kv heads then advances the item's length. Every workgroup of the
// grid reaches this point exactly once, which returns the counters to zero.
// With more outputs than threads, a thread merges EPT outputs of one row per
// pass, with the partial loads of all EPT outputs issued together: a batch of
// up to 16 partials costs one dependent memory round trip per pass instead
// of one per output (8 rows x D 256: 1 pass instead of 8). EPT is 8 where the
// decode already holds ~200 VGPRs (D >= 256, >= 2048 outputs), 2 elsewhere,
// so the tail does not raise a lighter kernel's register count. With at most
// one output per thread (the talker's 2 rows x D 128) each thread merges its
// own output (one round trip; the paired form measured 0.15 us slower per
// launch there). Per output the arithmetic is merge_partials<1>'s (batches of
// 16 in partial order), so both merge paths round identically.
template <int D, int R>
__device__ __forceinline__ void decode_merge_tail(const DecodeArgs &a, int item, int kvh, int hkv, int rows) {
    __shared__ uint32_t arrived;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are complete
    __syncthreads();
    uint32_t *hc = a.cnt + item * hkv + kvh;
    if (threadIdx.x == 0) arrived = arrive_agent(hc);
    __syncthreads();
    if (arrived != gridDim.x - 1) return;
    const int n_parts = gridDim.x;
    const int Qn = a.qn;
    const int64_t pbase = ((int64_t)item * hkv + kvh) * a.n_split * R;  // part s, row r at pbase + s*R + r
    if constexpr (R * D <= 256) {
        const int idx = threadIdx.x;
        if (idx < rows * D) {
            const int r = idx / D, d = idx % D;
            const float2 *ml = a.part_ml + pbase + r;
            const float *acc = a.part_acc + (pbase + r) * D + d;
            float M = kNegBig, L = 0.f, O = 0.f;
            merge_partials<1>(0, n_parts, [&](int sp, float2 &m, float &v) {
                m = load_agent(ml + (int64_t)sp * R);
                v = load_agent(acc + (int64_t)sp * R * D);
            }, M, L, O);
            // row r is q head kvh*g + r / Qn, query r % Qn
            a.out[(((int64_t)item * hkv * a.group + kvh * a.group) * Qn + r) * D + d] =
                f32_to_bf16(L > 0.f ? O / L : 0.f);
        }
    } else {
        constexpr int EPT = (D >= 256 && R * D >= 2048) ? 8 : 2;  // divides D (>= 64)
        constexpr int B = 16;
        // The D / EPT threads of a row take float2 columns j, j + D/EPT, ... so
        // that each load instruction reads whole consecutive runs of a row.
        constexpr int TPR = D / EPT;  // threads per row
        for (int e0 = threadIdx.x * EPT; e0 < rows * D; e0 += blockDim.x * EPT) {
            const int r = e0 / D, j = (e0 % D) / EPT;
            const float2 *ml = a.part_ml + pbase + r;
            const float2 *acc = reinterpret_cast<const float2 *>(a.part_acc + (pbase + r) * D) + j;
            float M = kNegBig, L = 0.f, O[EPT];
#pragma unroll
            for (int e = 0; e < EPT; ++e) O[e] = 0.f;
            for (int s0 = 0; s0 < n_parts; s0 += B) {
                float2 m[B], v[B][EPT / 2];
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    const int sp = s0 + u;
                    m[u] = make_float2(kNegBig, 0.f);
#pragma unroll
                    for (int h = 0; h < EPT / 2; ++h) v[u][h] = make_float2(0.f, 0.f);
                    if (sp < n_parts) {
                        m[u] = load_agent(ml + (int64_t)sp * R);
#pragma unroll
                        for (int h = 0; h < EPT / 2; ++h) v[u][h] = load_agent(acc + (int64_t)sp * R * D / 2 + h * TPR);
                    }
                }
                float bm = M;
#pragma unroll
                for (int u = 0; u < B; ++u) bm = fmaxf(bm, m[u].x);
                const float c = __builtin_amdgcn_exp2f(M - bm);
                L *= c;
#pragma unroll
                for (int e = 0; e < EPT; ++e) O[e] *= c;
                M = bm;
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    const float w = __builtin_amdgcn_exp2f(m[u].x - M);
                    L = fmaf(m[u].y, w, L);
#pragma unroll
                    for (int h = 0; h < EPT / 2; ++h) {
                        O[2 * h] = fmaf(v[u][h].x, w, O[2 * h]);
                        O[2 * h + 1] = fmaf(v[u][h].y, w, O[2 * h + 1]);
                    }
                }
            }
            // row r is q head kvh*g + r / Qn, query r % Qn
            const int64_t orow = (((int64_t)item * hkv * a.group + kvh * a.group) * Qn + r) * D;
            uint32_t *dst = reinterpret_cast<uint32_t *>(a.out + orow) + j;
#pragma unroll
            for (int h = 0; h < EPT / 2; ++h)
                dst[h * TPR] = (uint32_t)f32_to_bf16(L > 0.f ? O[2 * h] / L : 0.f) |
                               ((uint32_t)f32_to_bf16(L > 0.f ? O[2 * h + 1] / L : 0.f) << 16);
        }
    }
    if (threadIdx.x == 0) {
        clear_agent(hc);
        if (a.advance) {
            // every workgroup of the item has read its length by now
            uint32_t *ic = a.cnt + kCntItemBase + item;
            if (arrive_agent(ic) == (uint32_t)hkv - 1) {
                clear_agent(ic);
                a.len.lens[(int64_t)a.slots[item] * a.len.stride + a.len.offset] += Qn;
            }
        }
    }
}

template <int D, int R>
struct DecodeLds {
    static constexpr bool kWgMerge = decode_wg_merge(D, R);
    static constexpr int kFloats = kWgMerge ? kWaves * R * D : 1;
};

// grid (n_split / kWaves, kv_heads, n_items), 256 threads = kWaves waves.
// Wave w of workgroup x owns key split s = x*kWaves + w: a contiguous key
// range. Inside a wave, LPR = D/VEC lanes share one key row (VEC elements =
// 16 B each) and KPW = 64/LPR key rows are in flight per load instruction.
// The R rows of a kv head are its g q heads x Q query positions
// (row r = j*Q + i for q head kvh*g + j, query i).
// Args is DecodeArgs (causal / sliding-window visibility) or TalkerArgs (the
// talker's per-item prefix / audio ranges, bf16 CONTIG layers only).
//
// K/V reach the waves in one of two ways. DMA (bf16 CONTIG / RING, R <= 4):
// every wave streams its key range through its own LDS ring of kDmaStages
// stages x U key groups (K and V, 1 KiB each per group) plus its q rows; at
// pass p it waits for stage p, reads it into registers, refills it with pass
// p + kDmaStages and computes, so kDmaStages - 1 stages stay in flight during
// the arithmetic. Otherwise (int8, PAGED, more rows): a pass loads its U
// groups straight into registers, all before the first is used.
template <int D, int R, int KDT, int LAYOUT, class Args = DecodeArgs>
__global__ __launch_bounds__(256) void decode_kernel(Args a) {
    constexpr bool TALK = !std::is_same<Args, DecodeArgs>::value;
    static_assert(!TALK || (KDT == KVRT_BF16 && LAYOUT == KVRT_LAYOUT_CONTIG), "talker: bf16 CONTIG");
    constexpr int VEC = (KDT == KVRT_INT8) ? 16 : 8;
    constexpr int LPR = D / VEC;
    constexpr int KPW = 64 / LPR;
    constexpr bool DMA = decode_dma(R, KDT, LAYOUT, D);
    constexpr int U = decode_unroll(R, KDT, LAYOUT, D);
    constexpr int QW = VEC / 2;  // packed bf16 pairs of q per lane and row
    static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "bad head_dim");
    constexpr int STG = kDmaStages;
    constexpr int QI = (R * LPR + 63) / 64;                  // q DMA instructions per wave
    constexpr int WAVE_BYTES = DMA ? dma_wave_bytes(R, D) : 16;
    static_assert(!DMA || WAVE_BYTES == (STG * U * 2 + QI) * 1024, "ring layout");
    static_assert(!DMA || (STG >= 1 && 2 * U * STG < 64), "DMA ring: outstanding loads fit vmcnt");
    static_assert(!DMA || R * D * 4 <= WAVE_BYTES, "DMA ring holds the wave's partial");

    const int lane = threadIdx.x & 63;
    // wave-uniform (an SGPR): the split, key range and pass count follow
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = lane / LPR;
    const int seg = lane % LPR;
    // workgroups start in linear id order, z slowest: PAGED items (pools of
    // ragged sessions) come sorted by visible keys, longest first, so the
    // grid ends on short ones; other layouts keep z (the indirection is a
    // dependent argument load ahead of every workgroup's first load: +1 % on
    // the north-star step, whose items are equally long)
    const int item = LAYOUT == KVRT_LAYOUT_PAGED ? launch_item(a, blockIdx.z) : (int)blockIdx.z;
    const int kvh = blockIdx.y;
    const int hkv = gridDim.y;
    const int split = blockIdx.x * kWaves + wave;
    const int slot = a.slots[item];
    const int64_t new_base = (((int64_t)item * hkv + kvh) * a.qn) * D + seg * VEC;
    // wave-uniform (an SGPR): the key range, pass count and their tests follow
    const int len = __builtin_amdgcn_readfirstlane(a.len.lens[(int64_t)slot * a.len.stride + a.len.offset]);
    int plen = 0;          // prefix-attention mask (listener slots); the talker has its own masks
    uint32_t pw = ~0u;
    if constexpr (!TALK) load_prefix(a.pmask, slot, lane, plen, pw);
    const int Qn = a.qn;
    const int rows = a.group * Qn;
    const bool fused = a.k_new != nullptr;  // bf16: rows copied; int8: quantised in-kernel
    int kend = fused ? len + Qn : len;
    if constexpr (TALK) kend = min(kend, a.talk[item].audio_pos + 1);
    if (LAYOUT == KVRT_LAYOUT_CONTIG && kend > a.kv.rows) {
        // a length beyond the rows of the view (caller-provided lengths):
        // clamp the reads and raise the device flag
        if (threadIdx.x == 0 && blockIdx.x == 0) a.err[0] = 1;
        kend = a.kv.rows;
    }
    const int p0 = kend - Qn;
    const int kstart = a.window > 0 ? max(0, p0 - a.window + 1) : 0;
    const int nk = max(0, kend - kstart);
    int chunk = (nk + a.n_split - 1) / a.n_split;
    chunk = (chunk + KPW - 1) / KPW * KPW;
    const int ws = kstart + split * chunk;
    const int we = min(kend, ws + chunk);

    if constexpr (!TALK) apply_page_edits(a);
    if constexpr (KDT == KVRT_BF16) {
        // Fused append: workgroup 0 of every (item, kv head) stores the new
        // rows. No workgroup of this launch reads those cache rows (they are
        // taken from k_new below); RING rows overwritten here hold positions
        // older than the window.
        if (fused && blockIdx.x == 0) {
            for (int c = threadIdx.x; c < Qn * (D / 8); c += blockDim.x) {
                const int r = c / (D / 8), sg = c % (D / 8);
                const int pos = len + r;
                bool ok = true;
                if constexpr (LAYOUT == KVRT_LAYOUT_CONTIG) ok = pos < a.kv.rows;
                const int64_t dst = ok ? new_row_offset<LAYOUT>(a, slot, kvh, pos, D) : -1;
                if (dst < 0) {
                    a.err[0] = 1;
                    continue;
                }
                const int64_t src = (((int64_t)item * hkv + kvh) * Qn + r) * D + sg * 8;
                const uint4 kx = *reinterpret_cast<const uint4 *>(a.k_new + src);
                const uint4 vx = *reinterpret_cast<const uint4 *>(a.v_new + src);
                store_agent16(static_cast<uint16_t *>(a.kv.k) + dst + sg * 8, kx);
                store_agent16(static_cast<uint16_t *>(a.kv.v) + dst + sg * 8, vx);
            }
        }
    }

    // Fused int8 append. A wave whose key range reaches the new rows
    // quantises them (exactly as the append kernel does: LPR lanes of 16
    // values per row) into LDS before its main loop, where registers are
    // free, for the pass that reaches them; the one whose range starts at or
    // before the first of them also stores them with their scales (no
    // workgroup of the launch reads those cache rows). Two waves of a
    // workgroup may both fill the LDS copy: they write the same bytes, and
    // each reads its own writes. (The rows are loaded here rather than next
    // to the length load: holding them from there raised the kernel to 132
    // VGPRs, 3 waves per SIMD, and config 5 from 0.83 to 0.94 ms per step.)
    constexpr int NQ = KDT == KVRT_INT8 ? kMaxInt8Rows : 1;
    __shared__ uint4 nrow_k[NQ * LPR], nrow_v[NQ * LPR];
    __shared__ float nrow_s[2 * NQ];
    if constexpr (KDT == KVRT_INT8) {
        if (fused && we > len)
            i8_new_rows<D, NQ, LAYOUT>(a, item, slot, kvh, hkv, len, Qn, lane, ws <= len, nrow_k, nrow_v, nrow_s);
    }

    // q rows of this kv head, packed bf16 pairs. Row r = j*Q + i of the tile
    // is query i of q head kvh*g + j; rows past the real ones (r >= rows) load
    // row 0 and are never used (no key is visible to them), so the loads issue
    // back to back with no branch (a branch around a load makes the compiler
    // wait for it at the join, before the K/V loads are issued).
    uint32_t qw[R][QW];
    const int hq = hkv * a.group;
    if constexpr (!DMA) {  // DMA: staged through LDS below
        const uint16_t *q0 = a.q + ((int64_t)item * hq + kvh * a.group) * Qn * D + seg * VEC;
        int j = 0, i = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint16_t *qp = q0 + (r < rows ? (int64_t)(j * Qn + i) * D : 0);
#pragma unroll
            for (int t = 0; t < VEC / 8; ++t) {
                const uint4 x = *reinterpret_cast<const uint4 *>(qp + t * 8);
                qw[r][4 * t + 0] = x.x; qw[r][4 * t + 1] = x.y;
                qw[r][4 * t + 2] = x.z; qw[r][4 * t + 3] = x.w;
            }
            if (++i == Qn) {
                i = 0;
                ++j;
            }
        }
    }
    // Per-row visibility: key in [lo_r, hi_r]; talker rows add the audio
    // range [alo_r, ahi_r] and the gate gb_r over [blo, bhi].
    int hi[R], lo[R], alo[R], ahi[R];
    float gb[R];
    int blo = 0, bhi = -1;
    if constexpr (TALK) {
        const TalkerItem t = a.talk[item];
        blo = t.prefix_start;
        bhi = t.prefix_pos;
        const int base_hi = max(t.prefix_pos, t.prefix_start - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool audio = umod_uniform(r, Qn) == Qn - 1;
            lo[r] = 0;
            hi[r] = r >= rows ? -1 : (audio && t.mode == 1 ? t.prefix_start - 1 : base_hi);
            alo[r] = r < rows && audio ? t.audio_start : 0x7fffffff;
            ahi[r] = r < rows && audio ? t.audio_pos : -1;
            gb[r] = audio && t.mode == 2 ? t.gate_log2 : 0.f;
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int p = p0 + umod_uniform(r, Qn);
            hi[r] = r < rows ? p : -1;
            lo[r] = a.window > 0 ? p - a.window + 1 : 0;
            alo[r] = 0x7fffffff;
            ahi[r] = -1;
            gb[r] = 0.f;
        }
    }

    float m_run[R], l_run[R], acc[R][VEC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m_run[r] = kNegBig;
        l_run[r] = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[r][e] = 0.f;
    }

    bool bad = false;  // a visible key on an unmapped page (PAGED)
    const int npass = we > ws ? (we - ws + KPW * U - 1) / (KPW * U) : 0;
    // PAGED: the page-table entries of the wave's first 64 pages, one per
    // lane, so that a pass finds its pages with a lane shuffle instead of a
    // dependent global load
    int pwin = -1, pwin0 = 0;
    if constexpr (LAYOUT == KVRT_LAYOUT_PAGED) {
        pwin0 = ws >> a.kv.block_shift;
        pwin = load_page_window(a.kv, slot, pwin0, lane);
    }
    // PAGED: row offset of key kc >= base of the pass at base (-1: unmapped
    // page). The pass's keys, [base, min(we, base + KPW * U)), are looked up
    // in the wave's window of 64 page-table entries, which moves (a
    // wave-uniform branch) when a pass leaves it; a pass over more than 64
    // pages (tiny pages) looks them up directly. Every lane calls it together.
    // The lookups of a pass come before its K/V loads: a page-table load
    // between them would hold every later load of the pass until all earlier
    // ones had landed (a load's result is awaited by count, and loads
    // complete in order).
    auto pass_window = [&](int base) __attribute__((always_inline)) {
        const int lp_end = (min(we, base + KPW * U) - 1) >> a.kv.block_shift;
        if (lp_end - pwin0 >= 64) {
            pwin0 = base >> a.kv.block_shift;
            pwin = load_page_window(a.kv, slot, pwin0, lane);
        }
        return lp_end - pwin0 < 64;  // wave-uniform
    };
    auto page_off = [&](int kc, bool inwin) __attribute__((always_inline)) {
        const int lp = kc >> a.kv.block_shift;
        int page = __shfl(pwin, (lp - pwin0) & 63);
        if (!inwin) page = lp < a.kv.pt_stride ? a.kv.page_table[(int64_t)slot * a.kv.pt_stride + lp] : -1;
        return page_row_offset(a.kv, page, kvh, kc, D);
    };
    __shared__ __align__(16) u32x4_t dma_lds[DMA ? kWaves * WAVE_BYTES / 16 : 1];
    // this wave's LDS: q rows (QI KiB), then STG stages of U x (K, V) KiB
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t ring = lds_addr(dma_lds) + wave_u * WAVE_BYTES;
    const u32x4_t *ring_v = dma_lds + wave_u * (WAVE_BYTES / 16);
    // DMA of the U key groups of pass p into stage st (same addressing and
    // clamping as the register load below; CONTIG / RING rows always exist).
    auto dma_pass = [&](int p, int st) __attribute__((always_inline)) {
        const uint32_t dst = __builtin_amdgcn_readfirstlane(ring + (QI + st * U * 2) * 1024);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = ws + p * KPW * U + u * KPW + sub;
            const int kc = kk < we ? kk : ws;
            const int64_t o = row_offset<LAYOUT>(a.kv, slot, kvh, kc, D);
            const uint16_t *kp = static_cast<const uint16_t *>(a.kv.k) + o + seg * VEC;
            const uint16_t *vp = static_cast<const uint16_t *>(a.kv.v) + o + seg * VEC;
            if (fused) {
                const bool nw = kc >= len;
                const int64_t on = new_base + (int64_t)(kc - len) * D;
                kp = nw ? a.k_new + on : kp;
                vp = nw ? a.v_new + on : vp;
            }
            dma_load16(kp, dst + u * 2048);
            dma_load16(vp, dst + u * 2048 + 1024);
        }
    };
    if constexpr (DMA) {
        // q first (row r = e / LPR of element chunk e = t*64 + lane; rows past
        // the tile's real rows read row 0), then the first STG passes.
#pragma unroll
        for (int t = 0; t < QI; ++t) {
            const int e = t * 64 + lane;
            int r = e / LPR;
            r = r < rows ? r : 0;
            const uint16_t *qp = a.q + (((int64_t)item * hq + kvh * a.group) * Qn + r) * D + (e % LPR) * VEC;
            dma_load16(qp, __builtin_amdgcn_readfirstlane(ring + t * 1024));
        }
        const int pro = min(STG, npass);
        for (int p = 0; p < pro; ++p) dma_pass(p, p);
        wait_vmem_steps<2 * U, STG>(pro);  // q has landed
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32x4_t x = ring_v[r * LPR + seg];
            qw[r][0] = x[0]; qw[r][1] = x[1]; qw[r][2] = x[2]; qw[r][3] = x[3];
            if (r >= rows) qw[r][0] = qw[r][1] = qw[r][2] = qw[r][3] = 0u;
        }
    }
    for (int p = 0; p < npass; ++p) {
        const int base = ws + p * KPW * U;
        uint4 kx[U], vx[U];
        float ksc[U], vsc[U];
        int key[U];
        int64_t po[U];  // PAGED: row offsets of the pass's keys (-1: unmapped page)
        if constexpr (LAYOUT == KVRT_LAYOUT_PAGED) {
            const bool inwin = pass_window(base);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int kk = base + u * KPW + sub;
                po[u] = page_off(kk < we ? kk : base, inwin);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (DMA) {
            // stage p: wait for it (the later passes stay in flight), read it,
            // then refill the stage with pass p + STG before computing
            const int st = p % STG;
            wait_vmem_steps<2 * U, STG - 1>(min(STG - 1, npass - 1 - p));
            const u32x4_t *sv = ring_v + (QI * 1024 + st * U * 2048) / 16;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const u32x4_t x = sv[u * 128 + lane], y = sv[u * 128 + 64 + lane];
                kx[u] = make_uint4(x[0], x[1], x[2], x[3]);
                vx[u] = make_uint4(y[0], y[1], y[2], y[3]);
                const int kk = base + u * KPW + sub;
                key[u] = kk < we ? kk : 0x7fffffff;
                ksc[u] = vsc[u] = 0.f;
            }
            wait_lds();
            if (p + STG < npass) dma_pass(p + STG, st);
        } else {
        // Load phase, branch-free so that all 2U loads issue back to back:
        // a key past the wave's range (or on an unmapped page) reads a valid
        // row instead (the wave's first key / pool page 0) and is masked out
        // of the softmax; fused rows >= len come from the new K/V by an
        // address select.
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = base + u * KPW + sub;
            const int kc = kk < we ? kk : base;  // clamped: always a readable row
            int64_t o;
            if constexpr (LAYOUT == KVRT_LAYOUT_PAGED) o = po[u];
            else o = row_offset<LAYOUT>(a.kv, slot, kvh, kc, D);
            bool ok = kk < we;
            if constexpr (LAYOUT == KVRT_LAYOUT_PAGED) {
                // a fused append's new rows come from k_new / v_new; their
                // page may be mapped by this very launch
                const bool nw = fused && kc >= len;
                bad |= ok && !nw && o < 0;
                ok = ok && (nw || o >= 0);
                o = o < 0 ? 0 : o;
            }
            key[u] = ok ? kk : 0x7fffffff;
            if constexpr (KDT == KVRT_BF16) {
                const uint16_t *kp = static_cast<const uint16_t *>(a.kv.k) + o + seg * VEC;
                const uint16_t *vp = static_cast<const uint16_t *>(a.kv.v) + o + seg * VEC;
                if (fused) {
                    const bool nw = kc >= len;
                    const int64_t on = new_base + (int64_t)(kc - len) * D;
                    kp = nw ? a.k_new + on : kp;
                    vp = nw ? a.v_new + on : vp;
                }
                kx[u] = load_stream16(kp);
                vx[u] = load_stream16(vp);
                ksc[u] = vsc[u] = 0.f;
            } else {
                kx[u] = load_stream16(static_cast<const int8_t *>(a.kv.k) + o + seg * VEC);
                vx[u] = load_stream16(static_cast<const int8_t *>(a.kv.v) + o + seg * VEC);
                ksc[u] = a.kv.ks[o / D];
                vsc[u] = a.kv.vs[o / D];
            }
        }
        // keep all 2U loads of the pass ahead of the arithmetic (the scheduler
        // would otherwise sink the last ones under register pressure and
        // expose a second memory round trip per pass)
        __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (KDT == KVRT_INT8) {
            // Fused int8 append: the pass that reaches the new rows (one per
            // (item, kv head); wave-uniform) takes them, quantised, from LDS,
            // so the launch attends over the rows an append followed by a
            // decode would read.
            if (fused && base + KPW * U > len) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int kk = base + u * KPW + sub;
                    if (kk < we && kk >= len) {
                        const int r = kk - len;
                        kx[u] = nrow_k[r * LPR + seg];
                        vx[u] = nrow_v[r * LPR + seg];
                        ksc[u] = nrow_s[r];
                        vsc[u] = nrow_s[NQ + r];
                    }
                }
            }
        }
        if (base < plen) {
            // keys of this pass below the end of the prefix mask: a masked
            // key becomes invisible to every row (wave-uniform branch)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool hidden = key[u] < plen && !prefix_bit(pw, key[u]);
                key[u] = hidden ? 0x7fffffff : key[u];
            }
        }
        // scores (log2 domain)
        float s[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t kw[4] = {kx[u].x, kx[u].y, kx[u].z, kx[u].w};
            float kf[16];
            if constexpr (KDT == KVRT_INT8) {
#pragma unroll
                for (int e = 0; e < 16; ++e) kf[e] = (float)(int8_t)(kw[e >> 2] >> (8 * (e & 3)));
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float d = 0.f;
                if constexpr (KDT == KVRT_BF16) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) d = dot2_bf16(qw[r][t], kw[t], d);
                } else {
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        d = fmaf(bf16_lo(qw[r][t]), kf[2 * t], d);
                        d = fmaf(bf16_hi(qw[r][t]), kf[2 * t + 1], d);
                    }
                }
                d = group_sum<LPR>(d);
                if constexpr (KDT == KVRT_INT8) d *= ksc[u];
                if constexpr (TALK) {
                    const bool vis = key[u] <= hi[r] || (key[u] >= alo[r] && key[u] <= ahi[r]);
                    const bool gated = key[u] >= blo && key[u] <= bhi;
                    s[u][r] = vis ? fmaf(d, a.scale_log2, gated ? gb[r] : 0.f) : -INFINITY;
                } else {
                    const bool vis = key[u] <= hi[r] && key[u] >= lo[r];
                    s[u][r] = vis ? d * a.scale_log2 : -INFINITY;
                }
            }
        }
        // online softmax, one update per block of U keys; int8 decodes keep a
        // lazy running max (they are VALU-bound: the skipped rescales are ~9 %
        // of their instructions; config 5 32.8 -> 31.4 us), bf16 ones update
        // it every block (the branch slowed the bandwidth-bound talker launch
        // by 0.4 us and the sliding-window one by the same)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float mb = s[0][r];
#pragma unroll
            for (int u = 1; u < U; ++u) mb = fmaxf(mb, s[u][r]);
            if constexpr (KDT == KVRT_INT8) {
                if (mb > m_run[r] + kRescaleSlack) {
                    const float corr = __builtin_amdgcn_exp2f(m_run[r] - mb);
                    m_run[r] = mb;
                    l_run[r] *= corr;
#pragma unroll
                    for (int e = 0; e < VEC; ++e) acc[r][e] *= corr;
                }
            } else {
                const float mn = fmaxf(m_run[r], mb);
                const float corr = __builtin_amdgcn_exp2f(m_run[r] - mn);
                m_run[r] = mn;
                l_run[r] *= corr;
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[r][e] *= corr;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t vw[4] = {vx[u].x, vx[u].y, vx[u].z, vx[u].w};
            float vf[VEC];
            if constexpr (KDT == KVRT_BF16) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    vf[2 * t] = bf16_lo(vw[t]);
                    vf[2 * t + 1] = bf16_hi(vw[t]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e) vf[e] = (float)(int8_t)(vw[e >> 2] >> (8 * (e & 3)));
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float p = __builtin_amdgcn_exp2f(s[u][r] - m_run[r]);
                l_run[r] += p;
                if constexpr (KDT == KVRT_INT8) p *= vsc[u];
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[r][e] = fmaf(p, vf[e], acc[r][e]);
            }
        }
    }

    if constexpr (DMA) wait_vmem<0>();  // every DMA of this wave has landed (q too)
    if (bad) a.err[0] = 1;

    // merge the KPW key sub-groups of the wave (lanes LPR apart)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if constexpr (KPW > 1) {
            const float M = strided_max<LPR>(m_run[r]);
            const float w = __builtin_amdgcn_exp2f(m_run[r] - M);
            l_run[r] = strided_sum<LPR>(l_run[r] * w);
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[r][e] = strided_sum<LPR>(acc[r][e] * w);
            m_run[r] = M;
        }
    }
    using Lds = DecodeLds<D, R>;
    __shared__ __align__(16) float lds_own[DMA ? 1 : Lds::kFloats];
    __shared__ float2 lds_ml[kWaves * R];
    // a wave's partial: its own slice of lds_own, or (DMA) its own ring, which
    // it no longer reads or loads into
    float *lds = DMA ? reinterpret_cast<float *>(dma_lds) : lds_own;
    constexpr int PST = DMA ? WAVE_BYTES / 4 : R * D;  // floats between waves' partials
    if constexpr (Lds::kWgMerge) {
        // Workgroup merge: every wave puts its partial in LDS; wave w then
        // merges rows w, w + kWaves, ... over the kWaves partials (64 lanes
        // across D) and writes the workgroup's partial of those rows.
        if (sub == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float4 *dst = reinterpret_cast<float4 *>(lds + wave * PST + r * D + seg * VEC);
#pragma unroll
                for (int t = 0; t < VEC / 4; ++t)
                    dst[t] = make_float4(acc[r][4 * t], acc[r][4 * t + 1], acc[r][4 * t + 2], acc[r][4 * t + 3]);
                if (seg == 0) lds_ml[wave * R + r] = make_float2(m_run[r], l_run[r]);
            }
        }
        __syncthreads();
        constexpr int EPL = D / 64;  // dims per lane
        const int64_t pbase = (((int64_t)item * hkv + kvh) * a.n_split + blockIdx.x) * R;
        for (int r = wave; r < R && r < rows; r += kWaves) {
            float M = kNegBig;
#pragma unroll
            for (int w2 = 0; w2 < kWaves; ++w2) M = fmaxf(M, lds_ml[w2 * R + r].x);
            float L = 0.f, o[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) o[e] = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < kWaves; ++w2) {
                const float2 ml = lds_ml[w2 * R + r];
                const float ww = __builtin_amdgcn_exp2f(ml.x - M);
                L = fmaf(ml.y, ww, L);
                const float *src = lds + w2 * PST + r * D + lane * EPL;
#pragma unroll
                for (int e = 0; e < EPL; ++e) o[e] = fmaf(src[e], ww, o[e]);
            }
            float *dst = a.part_acc + (pbase + r) * D + lane * EPL;
            if (a.cnt) {
                store_agent_n<EPL>(dst, o);
                if (lane == 0) store_agent(a.part_ml + pbase + r, make_float2(M, L));
            } else {
#pragma unroll
                for (int e = 0; e < EPL; ++e) dst[e] = o[e];
                if (lane == 0) a.part_ml[pbase + r] = make_float2(M, L);
            }
        }
        if (a.cnt) decode_merge_tail<D, R>(a, item, kvh, hkv, rows);
    } else if (sub == 0) {
        // one partial per wave
        const int64_t pbase = (((int64_t)item * hkv + kvh) * a.n_split + split) * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r < rows) {
                float4 *dst = reinterpret_cast<float4 *>(a.part_acc + (pbase + r) * D + seg * VEC);
#pragma unroll
                for (int t = 0; t < VEC / 4; ++t)
                    dst[t] = make_float4(acc[r][4 * t], acc[r][4 * t + 1], acc[r][4 * t + 2], acc[r][4 * t + 3]);
                if (seg == 0) a.part_ml[pbase + r] = make_float2(m_run[r], l_run[r]);
            }
        }
    }
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16k16(uint2 a, uint2 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b),
                                                     c, 0, 0, 0);
}
// Online-softmax update of an MFMA accumulator column with a lazy reference
// max (kRescaleSlack): the l / o rescale (o lives in AGPRs: a read, multiply
// and write per element) runs a few times per wave instead of on most tiles.
template <int NB>
__device__ __forceinline__ void lazy_rescale(float tmax, float &m, float &l, f32x4_t (&o)[NB]) {
    if (tmax > m + kRescaleSlack) {
        if (m != kNegBig) {  // otherwise nothing has been accumulated yet
            const float corr = __builtin_amdgcn_exp2f(m - tmax);
            l *= corr;
#pragma unroll
            for (int b = 0; b < NB; ++b) o[b] *= corr;
        }
        m = tmax;
    }
}

// gfx950 LDS transpose read: in each group of 16 lanes, lane s gives the
// address of 4 consecutive bf16; lane t = 4a + e receives element e of the
// chunks of lanes a, a + 4, a + 8, a + 12.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p) {
    const s16x4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s16x4_t __attribute__((address_space(3))) *)(p));
    return __builtin_bit_cast(uint2, x);
}

// Split-K decode on MFMA for R = g*Q in {8, 16} query rows per kv head
// (bf16): same grid, key splits, visibility and partial format as
// decode_kernel, one partial per workgroup. Per 16-key tile a wave computes
//   S^T (16 keys x 16 rows) = K Q^T   D/32 v_mfma_f32_16x16x32_bf16, K read
//                                     straight from HBM as the A operand
//   O^T (D x 16) += V^T P^T           2 * D/16 v_mfma_f32_16x16x16_bf16
// with the V tile staged row-major in the wave's own LDS slice and read
// transposed (ds_read_b64_tr_b16), and P as two bf16 terms. Lane layouts:
// 16x16x32 A[i l%16][k 8(l/16)+j], 16x16x16 A[i l%16][k 4(l/16)+j],
// B[k ..][n l%16], D[i 4(l/16)+v][n l%16]; column n is query row r.
// Four int8 values (one dword) as four bf16 (two packed dwords); exact, as
// every int8 value has at most 7 significant bits.
__device__ __forceinline__ uint2 i8x4_to_bf16(uint32_t w) {
    return make_uint2(pack_bf16x2((float)(int8_t)w, (float)(int8_t)(w >> 8)),
                      pack_bf16x2((float)(int8_t)(w >> 16), (float)(int8_t)(w >> 24)));
}

// Stages per wave of the MFMA decode's LDS DMA ring (mfma_decode_dma). A
// wave copies a stage into registers and refills it before computing, so
// with S stages S tiles are in flight during a tile's MFMAs. Two at D 128
// (72 KB per workgroup; 1, 3 and 4 stages: 0.598, 0.555 and 0.584 vs 0.542
// ms per two-stream step), one at D 256 (80 KB; two, 147 KB, ran the
// thinker's global layer faster alone but kept the talker's workgroups off
// its CUs: step 0.564 vs 0.542 ms).
#ifndef KVRT_MFMA_DMA_STAGES_128
#define KVRT_MFMA_DMA_STAGES_128 2
#endif
#ifndef KVRT_MFMA_DMA_STAGES_256
#define KVRT_MFMA_DMA_STAGES_256 1
#endif
// Chunk swizzle of the MFMA decode's DMA tiles: the logical 16-byte chunk c
// of tile row r sits at chunk c ^ mfma_dswz(r), a permutation of the low 4
// bits that keeps bit 0 clear on rows 0-7. The K A-operand reads (16 rows,
// one chunk each, per 16 lanes) and the V^T transposed reads (4 rows x 2
// chunks x 2 halves per 16 lanes, 32 lanes per pass) then hit distinct
// banks (rows are 256 or 512 B: every row starts on bank 0).
__device__ __forceinline__ int mfma_dswz(int r) { return (2 * (r & 7)) ^ ((r >> 3) & 1); }

// The end of an MFMA decode workgroup. o holds its wave's O^T tile (o[b]:
// dims 16b + 4grp + v of row col), m the row's running max, l this lane's
// share of the row's sum. Every wave puts its partial in LDS (lds_raw, at
// least kWaves * R * (D + 4) floats, free of other use from here on); wave w
// then merges rows w, w + kWaves, ... and writes the workgroup's partial of
// those rows (one partial per workgroup, as decode_kernel), and with a merge
// counter the last workgroup of the (item, kv head) merges the partials.
template <int D, int R>
__device__ __forceinline__ void mfma_decode_finish(const DecodeArgs &a, uint8_t *lds_raw, float2 *lds_ml,
                                                   const f32x4_t (&o)[D / 16], float m, float l, int wave, int lane,
                                                   bool rvalid, int item, int kvh, int hkv, int rows) {
    // partial rows in LDS are PP floats apart: 16 B of padding per row, so the
    // 16 rows (query columns) of a half-wave's float4 writes start on distinct
    // banks (with a pitch of D floats they all hit the same ones)
    constexpr int PP = D + 4;
    const int col = lane & 15, grp = lane >> 4;
    l = pair<OpSum, 32>(pair<OpSum, 16>(l));
    __syncthreads();  // every wave is done with its tiles
    float *lds_part = reinterpret_cast<float *>(lds_raw);
    if (rvalid) {  // columns >= rows (>= R when R = 8) hold no row of this wave
        float *dst = lds_part + (wave * R + col) * PP + 4 * grp;
#pragma unroll
        for (int b = 0; b < D / 16; ++b)
            *reinterpret_cast<float4 *>(dst + 16 * b) = make_float4(o[b][0], o[b][1], o[b][2], o[b][3]);
        if (grp == 0) lds_ml[wave * R + col] = make_float2(m, l);
    }
    __syncthreads();
    constexpr int EPL = D / 64;  // dims per lane
    const int64_t pbase = (((int64_t)item * hkv + kvh) * a.n_split + blockIdx.x) * R;
    for (int r = wave; r < R && r < rows; r += kWaves) {
        float M = kNegBig;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; ++w2) M = fmaxf(M, lds_ml[w2 * R + r].x);
        float L = 0.f, acc[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; ++w2) {
            const float2 ml = lds_ml[w2 * R + r];
            const float ww = __builtin_amdgcn_exp2f(ml.x - M);
            L = fmaf(ml.y, ww, L);
            const float *src = lds_part + (w2 * R + r) * PP + lane * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[e] = fmaf(src[e], ww, acc[e]);
        }
        float *dst = a.part_acc + (pbase + r) * D + lane * EPL;
        if (a.cnt) {
            store_agent_n<EPL>(dst, acc);
            if (lane == 0) store_agent(a.part_ml + pbase + r, make_float2(M, L));
        } else {
#pragma unroll
            for (int e = 0; e < EPL; ++e) dst[e] = acc[e];
            if (lane == 0) a.part_ml[pbase + r] = make_float2(M, L);
        }
    }
    if (a.cnt) decode_merge_tail<D, R>(a, item, kvh, hkv, rows);
}

template <int D, int R, int LAYOUT, int KDT = KVRT_BF16>
__global__ __launch_bounds__(256) void decode_mfma_kernel(DecodeArgs a) {
    constexpr int T = kMfmaDecodeKeys;
    // V tile row pitch (bf16): rows 32 B apart modulo the 256 B of LDS banks, so
    // the 4 rows x 4 chunks of 8 B that 16 lanes of a transposed read touch
    // land on distinct banks (a 16 B shift made rows r and r + 1 overlap)
    constexpr int KP = D + 16;
    constexpr bool I8 = KDT == KVRT_INT8;
    static_assert(R == 8 || R == 16, "MFMA decode row tiles");
    static_assert(!I8 || LAYOUT == KVRT_LAYOUT_PAGED, "int8 rows are PAGED");
    // the waves' V tiles while streaming, their partials for the merge after
    // partial rows in LDS are PP floats apart: 16 B of padding per row, so the
    // 16 rows (query columns) of a half-wave's float4 writes start on distinct
    // banks (with a pitch of D floats they all hit the same ones)
    constexpr int PP = D + 4;
    constexpr int kTileBytes = kWaves * T * KP * 2, kPartBytes = kWaves * R * PP * 4;
    // DMA ring: per wave a copy of the tile's q rows (QB) and NSTG stages of
    // a K and a V tile (TB each), NSTG - 1 tiles in flight while one computes
    constexpr bool DMA = R == 8 && mfma_decode_dma(D, R, KDT, LAYOUT);
    constexpr int NSTG = D == 128 ? KVRT_MFMA_DMA_STAGES_128 : KVRT_MFMA_DMA_STAGES_256;
    constexpr int TB = T * D * 2, QB = R * D * 2;
    constexpr int DPT = 2 * TB / 1024;  // DMA instructions per tile (K and V)
    constexpr int kRingBytes = DMA ? kWaves * (QB + NSTG * 2 * TB) : 0;
    static_assert(!DMA || (NSTG >= 1 && DPT * NSTG < 64 && kRingBytes + kWaves * R * 8 <= 160 * 1024),
                  "DMA ring: outstanding loads fit vmcnt, the rings fit LDS");
    constexpr int kLdsBytes = kTileBytes > kPartBytes ? (kTileBytes > kRingBytes ? kTileBytes : kRingBytes)
                                                      : (kPartBytes > kRingBytes ? kPartBytes : kRingBytes);
    __shared__ __align__(16) uint8_t lds_raw[kLdsBytes];
    __shared__ float2 lds_ml[kWaves * R];
    uint16_t *sv_all = reinterpret_cast<uint16_t *>(lds_raw);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int item = LAYOUT == KVRT_LAYOUT_PAGED ? launch_item(a, blockIdx.z) : (int)blockIdx.z;
    const int kvh = blockIdx.y, hkv = gridDim.y;
    const int split = blockIdx.x * kWaves + wave;
    const int slot = a.slots[item];
    // The scalar arguments of the set-up, loaded in one batch with the slot
    // (one round trip) rather than each at its first use
    asm volatile("" ::"s"(a.qn), "s"(a.group), "s"(a.window), "s"(a.n_split), "s"(a.k_new), "s"(a.v_new),
                 "s"(a.kv.rows), "s"(a.pmask), "s"(a.q), "s"(a.kv.k), "s"(a.kv.v), "s"(a.kv.slot_stride),
                 "s"(a.kv.head_stride), "s"(a.len.lens), "s"(a.len.stride), "s"(a.len.offset), "s"(a.err),
                 "s"(a.n_upd), "s"(slot));
    const int len = a.len.lens[(int64_t)slot * a.len.stride + a.len.offset];
    // Prefix-attention mask of the slot. PAGED rows at D 512 use every
    // register: launches with masks run that shape on decode_kernel instead
    // (launch_decode_mfma refuses them), so this variant has no mask code.
    constexpr bool PMASK = !(LAYOUT == KVRT_LAYOUT_PAGED && D >= 512);
    int plen = 0;
    uint32_t pw = ~0u;
    if constexpr (PMASK) load_prefix(a.pmask, slot, lane, plen, pw);
    const int Qn = a.qn;
    const int rows = a.group * Qn;
    const bool fused = !I8 && a.k_new != nullptr;  // int8 rows are quantised by the append kernel
    int kend = fused ? len + Qn : len;
    if (LAYOUT == KVRT_LAYOUT_CONTIG && kend > a.kv.rows) {
        if (threadIdx.x == 0 && blockIdx.x == 0) a.err[0] = 1;
        kend = a.kv.rows;
    }
    const int p0 = kend - Qn;
    const int kstart = a.window > 0 ? max(0, p0 - a.window + 1) : 0;
    const int nk = max(0, kend - kstart);
    int chunk = (nk + a.n_split - 1) / a.n_split;
    chunk = (chunk + T - 1) / T * T;
    const int ws = kstart + split * chunk;
    const int we = min(kend, ws + chunk);

    // Fused append: workgroup 0 of every (item, kv head) stores the new rows;
    // no workgroup of this launch reads them from the cache.
    apply_page_edits(a);
    if (!I8 && fused && blockIdx.x == 0) {
        for (int c = threadIdx.x; c < Qn * (D / 8); c += blockDim.x) {
            const int r = c / (D / 8), sg = c % (D / 8);
            const int pos = len + r;
            bool ok = true;
            if constexpr (LAYOUT == KVRT_LAYOUT_CONTIG) ok = pos < a.kv.rows;
            const int64_t dst = ok ? new_row_offset<LAYOUT>(a, slot, kvh, pos, D) : -1;
            if (dst < 0) {
                a.err[0] = 1;
                continue;
            }
            const int64_t src = (((int64_t)item * hkv + kvh) * Qn + r) * D + sg * 8;
            const uint4 kx = *reinterpret_cast<const uint4 *>(a.k_new + src);
            const uint4 vx = *reinterpret_cast<const uint4 *>(a.v_new + src);
            store_agent16(static_cast<uint16_t *>(a.kv.k) + dst + sg * 8, kx);
            store_agent16(static_cast<uint16_t *>(a.kv.v) + dst + sg * 8, vx);
        }
    }

    // Q^T as the B operand: column col is row r = col (q head kvh*g + r/Qn,
    // query r % Qn); lane (col, grp) holds dims kdim(c) .. +7 of reduction
    // step c, K's A operand the same dims of its key: 32c + 8grp (bf16), or
    // 64(c/2) + 16grp + 8(c%2) for int8, so that a lane's two steps c, c + 1
    // are one 16-byte int8 load.
    auto kdim = [&](int c) { return I8 ? 64 * (c >> 1) + 16 * grp + 8 * (c & 1) : 32 * c + 8 * grp; };
    const int hq = hkv * a.group;
    const bool rvalid = col < rows;
    uint4 qop[D / 32];
    if constexpr (!DMA) {
        // every lane loads (rows past the tile's real rows read row 0), then
        // those lanes zero their operand: no branch around the loads
        // row col is q head kvh*g + col / Qn, query col % Qn
        const uint16_t *qp = a.q + (((int64_t)item * hq + kvh * a.group) * Qn + (rvalid ? col : 0)) * D;
#pragma unroll
        for (int c = 0; c < D / 32; ++c) qop[c] = *reinterpret_cast<const uint4 *>(qp + kdim(c));
#pragma unroll
        for (int c = 0; c < D / 32; ++c)
            if (!rvalid) qop[c] = make_uint4(0, 0, 0, 0);
    }
    const int cq = umod_uniform(col, Qn);  // this column's query
    const int hi = rvalid ? p0 + cq : -1;
    const int lo = a.window > 0 ? p0 + cq - a.window + 1 : 0;
    float m = kNegBig, l = 0.f;  // running max (uniform per column) and this lane's partial sum
    f32x4_t o[D / 16];
#pragma unroll
    for (int b = 0; b < D / 16; ++b) o[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint16_t *sv = sv_all + wave * (T * KP);
    const uint16_t *sv_lane = sv + (4 * grp + (col >> 2)) * KP + 4 * (col & 3);
    bool bad = false;
    const int64_t new_base = ((int64_t)item * hkv + kvh) * Qn * D;
    // PAGED below D 512: the page-table entries of the wave's first 64 pages,
    // one per lane, so that a tile finds its pages with a lane shuffle instead
    // of a dependent global load ahead of its K/V loads (at D 512 the window
    // does not fit the registers)
    constexpr bool PWIN = LAYOUT == KVRT_LAYOUT_PAGED && D < 512;
    int pwin = -1, pwin0 = 0;
    if constexpr (PWIN) {
        pwin0 = ws >> a.kv.block_shift;
        pwin = load_page_window(a.kv, slot, pwin0, lane);
    }
    // PWIN: the window moves (a wave-uniform branch, before the tile's
    // loads) when the tile at t0 leaves it; a tile spans at most T pages, so
    // the window then covers it, and no page-table load sits between K/V
    // loads (its wait would hold every later load until all earlier ones
    // had landed)
    auto tile_window = [&](int t0) __attribute__((always_inline)) {
        if constexpr (PWIN) {
            if (((min(we, t0 + T) - 1) >> a.kv.block_shift) - pwin0 >= 64) {
                pwin0 = t0 >> a.kv.block_shift;
                pwin = load_page_window(a.kv, slot, pwin0, lane);
                asm volatile("" ::"v"(pwin));
            }
        }
    };
    // Row offset of key kk of the wave's range (keys past we read row ws, or
    // with PWIN a row of the window, and are masked).
    auto key_off = [&](int kk) __attribute__((always_inline)) {
        const int kc = kk < we ? kk : ws;
        int64_t off;
        if constexpr (PWIN)
            off = page_row_offset(a.kv, __shfl(pwin, ((kc >> a.kv.block_shift) - pwin0) & 63), kvh, kc, D);
        else
            off = row_offset<LAYOUT>(a.kv, slot, kvh, kc, D);
        if constexpr (LAYOUT == KVRT_LAYOUT_PAGED) {
            // a fused append's new rows come from k_new / v_new (their page
            // may be mapped by this very launch)
            bad |= kk < we && !(fused && kc >= len) && off < 0;
            off = off < 0 ? 0 : off;
        }
        return off;
    };
    // bf16 row addresses; the rows of a fused append come from k_new / v_new
    // (address selects under a uniform branch: a divergent branch here splits
    // the tile's loads and makes the compiler wait on the earlier ones)
    auto key_rows = [&](int kk, const uint16_t *&kp, const uint16_t *&vp) __attribute__((always_inline)) {
        const int64_t off = key_off(kk);
        kp = static_cast<const uint16_t *>(a.kv.k) + off;
        vp = static_cast<const uint16_t *>(a.kv.v) + off;
        if (fused) {
            const int kc = kk < we ? kk : ws;
            const bool nw = kc >= len;
            const int64_t on = new_base + (int64_t)(kc - len) * D;
            kp = nw ? a.k_new + on : kp;
            vp = nw ? a.v_new + on : vp;
        }
    };
    // The K and V loads of a tile, as loaded (KR / VR 16-byte units per
    // lane). bf16: K of the tile at t0 is the A operand (lane (col, grp): key
    // t0 + col, dims kdim(c)), V units u = lane + 64i (key row u / (D/8), 16 B
    // segment u % (D/8)). int8: K units of 16 dims (steps c, c + 1), V units
    // u of 16 values (key row u / (D/16)), plus the K and V scales of key
    // t0 + col; the tile converts them to bf16.
    constexpr int KR = I8 ? D / 64 : D / 32, VR = I8 ? D / 64 : D / 32;
    constexpr int VU = I8 ? D / 16 : D / 8;  // 16-byte units per V row
    auto load_k = [&](int t0, uint4 (&ka)[KR], float &ks, float &vs) __attribute__((always_inline)) {
        tile_window(t0);  // load_k comes first for every tile
        if constexpr (I8) {
            const int64_t off = key_off(t0 + col);
            const int8_t *kp = static_cast<const int8_t *>(a.kv.k) + off;
#pragma unroll
            for (int c2 = 0; c2 < KR; ++c2) ka[c2] = load_stream16(kp + kdim(2 * c2));
            ks = a.kv.ks[off / D];
            vs = a.kv.vs[off / D];
        } else {
            const uint16_t *kp, *vp;
            key_rows(t0 + col, kp, vp);
#pragma unroll
            for (int c = 0; c < KR; ++c) ka[c] = load_stream16(kp + kdim(c));
        }
    };
    auto load_v = [&](int t0, uint4 (&vt)[VR]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < VR; ++i) {
            const int u = lane + 64 * i;
            if constexpr (I8) {
                const int64_t off = key_off(t0 + u / VU);
                vt[i] = load_stream16(static_cast<const int8_t *>(a.kv.v) + off + 16 * (u % VU));
            } else {
                const uint16_t *kp, *vp;
                key_rows(t0 + u / VU, kp, vp);
                vt[i] = load_stream16(vp + 8 * (u % VU));
            }
        }
    };
    if constexpr (!DMA) {
        // Software pipeline over the wave's tiles: tile t + 1's K is loaded into
        // the A-operand registers as soon as tile t's S MFMAs have read them, and
        // its V as soon as tile t's V is in LDS, so both are in flight during tile
        // t's softmax and P.V.
        // (PAGED at D 512 keeps one tile in flight: the page lookups of a second
        // tile do not fit the registers.)
        constexpr bool PIPE = !(LAYOUT == KVRT_LAYOUT_PAGED && D >= 512);
        uint4 ka[KR], vt[VR];
        float ksl = 0.f, vsl = 0.f;  // int8: scales of key t0 + col
        if (PIPE && ws < we) {
            load_k(ws, ka, ksl, vsl);
            load_v(ws, vt);
        }
        // The loop runs the tiles that have a successor with unconditional loads
        // of the next tile (a conditional load would make the compiler's wait
        // counts assume it may be missing, and wait on the next tile's first load
        // before storing this tile's V); the last tile is peeled.
        auto tile = [&](int t0, auto more_c) __attribute__((always_inline)) {
            constexpr bool more = PIPE && decltype(more_c)::value;
            if constexpr (!PIPE) {
                load_k(t0, ka, ksl, vsl);
                load_v(t0, vt);
            }
            f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
            float ksv[4], vsv[4];  // int8: K and V scales of this lane's keys t0 + 4grp + v
            if constexpr (I8) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    ksv[v] = __shfl(ksl, 4 * grp + v);
                    vsv[v] = __shfl(vsl, 4 * grp + v);
                }
#pragma unroll
                for (int c2 = 0; c2 < KR; ++c2) {
                    const uint2 a0 = i8x4_to_bf16(ka[c2].x), a1 = i8x4_to_bf16(ka[c2].y);
                    const uint2 a2 = i8x4_to_bf16(ka[c2].z), a3 = i8x4_to_bf16(ka[c2].w);
                    s = mfma16(make_uint4(a0.x, a0.y, a1.x, a1.y), qop[2 * c2], s);
                    s = mfma16(make_uint4(a2.x, a2.y, a3.x, a3.y), qop[2 * c2 + 1], s);
                }
            } else {
#pragma unroll
                for (int c = 0; c < KR; ++c) s = mfma16(ka[c], qop[c], s);
            }
            if constexpr (more) load_k(t0 + T, ka, ksl, vsl);
#pragma unroll
            for (int i = 0; i < VR; ++i) {
                const int u = lane + 64 * i;
                if constexpr (I8) {
                    const uint2 b0 = i8x4_to_bf16(vt[i].x), b1 = i8x4_to_bf16(vt[i].y);
                    const uint2 b2 = i8x4_to_bf16(vt[i].z), b3 = i8x4_to_bf16(vt[i].w);
                    uint4 *dst = reinterpret_cast<uint4 *>(sv + (u / VU) * KP + 16 * (u % VU));
                    dst[0] = make_uint4(b0.x, b0.y, b1.x, b1.y);
                    dst[1] = make_uint4(b2.x, b2.y, b3.x, b3.y);
                } else {
                    *reinterpret_cast<uint4 *>(sv + (u / VU) * KP + 8 * (u % VU)) = vt[i];
                }
            }
            if constexpr (more) load_v(t0 + T, vt);
            // this lane: keys t0 + 4grp + v of row col
            float sc[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int key = t0 + 4 * grp + v;
                const bool vis = key < we && key <= hi && key >= lo;
                sc[v] = vis ? (I8 ? s[v] * ksv[v] : s[v]) * a.scale_log2 : -INFINITY;
            }
            if (PMASK && t0 < plen) {  // the tile reaches into the prefix mask (wave-uniform)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int key = t0 + 4 * grp + v;
                    sc[v] = key < plen && !prefix_bit(pw, key) ? -INFINITY : sc[v];
                }
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; ++v) tmax = fmaxf(tmax, sc[v]);
            tmax = pair<OpMax, 32>(pair<OpMax, 16>(tmax));
            lazy_rescale<D / 16>(tmax, m, l, o);
            float p[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                p[v] = __builtin_amdgcn_exp2f(sc[v] - m);
                l += p[v];
                if constexpr (I8) p[v] *= vsv[v];  // dequantise V through P
            }
            // P = P_hi + P_lo in bf16 (as in the prefill kernel)
            const uint32_t h01 = pack_bf16x2(p[0], p[1]), h23 = pack_bf16x2(p[2], p[3]);
            const uint2 ph = make_uint2(h01, h23);
            const uint2 pl = make_uint2(pack_bf16x2(p[0] - bf16_lo(h01), p[1] - bf16_hi(h01)),
                                        pack_bf16x2(p[2] - bf16_lo(h23), p[3] - bf16_hi(h23)));
#pragma unroll
            for (int b = 0; b < D / 16; ++b) {
                const uint2 va = lds_read_tr16(sv_lane + 16 * b);
                o[b] = mfma16k16(va, pl, mfma16k16(va, ph, o[b]));
            }
        };
        int t0 = ws;
        for (; t0 + T < we; t0 += T) tile(t0, std::true_type{});
        if (t0 < we) tile(t0, std::false_type{});
    } else {
        // LDS DMA ring: each wave streams its q rows and then its 16-key K and V
        // tiles into its own LDS with global_load_lds_dwordx4 (16 B per lane,
        // 1 KiB = RPI rows per instruction; lane l fetches the logical chunk that
        // lands at chunk l % CPR of its row, see mfma_dswz), NSTG stages deep. A
        // tile's stage is copied into its operand registers and refilled with
        // the tile NSTG ahead before the tile's MFMAs, so NSTG tiles are in
        // flight while one is computed. The DMAs are invisible to the compiler's wait
        // counts: every wait is an explicit vmcnt on the wave's own DMAs, which
        // complete in issue order (q, tile 0, tile 1, ...). Rows past the wave's
        // range read row ws and are masked; fused rows come from k_new / v_new.
        constexpr int CPR = D / 8;     // 16-byte chunks per row
        constexpr int RPI = 64 / CPR;  // rows per DMA instruction
        const int wave_u = __builtin_amdgcn_readfirstlane(wave);
        const uint32_t ring = lds_addr(lds_raw) + wave_u * (kRingBytes / kWaves);
        const uint8_t *ring_p = lds_raw + wave_u * (kRingBytes / kWaves);
        const int ntiles = __builtin_amdgcn_readfirstlane(we > ws ? (we - ws + T - 1) / T : 0);
        auto dma_tile = [&](int j, int st) __attribute__((always_inline)) {
            const uint32_t kd = __builtin_amdgcn_readfirstlane(ring + QB + st * 2 * TB);
#pragma unroll
            for (int i = 0; i < TB / 1024; ++i) {
                const int row = RPI * i + lane / CPR;
                const int lc = (lane % CPR) ^ mfma_dswz(row);
                const uint16_t *kp, *vp;
                key_rows(ws + j * T + row, kp, vp);
                dma_load16(kp + 8 * lc, kd + i * 1024);
                dma_load16(vp + 8 * lc, kd + TB + i * 1024);
            }
        };
        {
            // q rows of the tile (rows past the real ones read row 0 and are
            // zeroed below), swizzled like the K tiles
#pragma unroll
            for (int i = 0; i < QB / 1024; ++i) {
                const int row = RPI * i + lane / CPR;
                const int lc = (lane % CPR) ^ mfma_dswz(row);
                const int rq = row < rows ? row : 0;
                const uint16_t *qp = a.q + (((int64_t)item * hq + kvh * a.group) * Qn + rq) * D;
                dma_load16(qp + 8 * lc, __builtin_amdgcn_readfirstlane(ring + i * 1024));
            }
        }
        const int pro = min(NSTG, ntiles);
        for (int j = 0; j < pro; ++j) dma_tile(j, j);
        wait_vmem_steps<DPT, NSTG>(pro);  // q has landed
#pragma unroll
        for (int c = 0; c < D / 32; ++c) {
            const int r8 = col & 7;  // columns >= R read row col - 8 and are zeroed
            qop[c] = *reinterpret_cast<const uint4 *>(ring_p + r8 * (D * 2) + 16 * ((4 * c + grp) ^ mfma_dswz(r8)));
            if (!rvalid) qop[c] = make_uint4(0, 0, 0, 0);
        }
        const int vrow = 4 * grp + (col >> 2);  // this lane's V^T read row
        for (int j = 0; j < ntiles; ++j) {
            const int st = j % NSTG;
            wait_vmem_steps<DPT, NSTG - 1>(min(NSTG - 1, ntiles - 1 - j));
            const uint8_t *kst = ring_p + QB + st * 2 * TB, *vst = kst + TB;
            uint4 kop[KR];
            uint2 vop[D / 16];
#pragma unroll
            for (int c = 0; c < KR; ++c)
                kop[c] = *reinterpret_cast<const uint4 *>(kst + col * (D * 2) + 16 * ((4 * c + grp) ^ mfma_dswz(col)));
#pragma unroll
            for (int b = 0; b < D / 16; ++b)
                vop[b] = lds_read_tr16(reinterpret_cast<const uint16_t *>(
                    vst + vrow * (D * 2) + 16 * ((2 * b + ((col & 3) >> 1)) ^ mfma_dswz(vrow)) + 8 * (col & 1)));
            wait_lds();  // the stage is in registers: refill it
            if (j + NSTG < ntiles) dma_tile(j + NSTG, st);
            const int t0 = ws + j * T;
            f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < KR; ++c) s = mfma16(kop[c], qop[c], s);
            float sc[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int key = t0 + 4 * grp + v;
                const bool vis = key < we && key <= hi && key >= lo;
                sc[v] = vis ? s[v] * a.scale_log2 : -INFINITY;
            }
            if (PMASK && t0 < plen) {  // the tile reaches into the prefix mask (wave-uniform)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int key = t0 + 4 * grp + v;
                    sc[v] = key < plen && !prefix_bit(pw, key) ? -INFINITY : sc[v];
                }
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; ++v) tmax = fmaxf(tmax, sc[v]);
            tmax = pair<OpMax, 32>(pair<OpMax, 16>(tmax));
            lazy_rescale<D / 16>(tmax, m, l, o);
            float p[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                p[v] = __builtin_amdgcn_exp2f(sc[v] - m);
                l += p[v];
            }
            // P = P_hi + P_lo in bf16, as in the register-staged tiles
            const uint32_t h01 = pack_bf16x2(p[0], p[1]), h23 = pack_bf16x2(p[2], p[3]);
            const uint2 ph = make_uint2(h01, h23);
            const uint2 pl = make_uint2(pack_bf16x2(p[0] - bf16_lo(h01), p[1] - bf16_hi(h01)),
                                        pack_bf16x2(p[2] - bf16_lo(h23), p[3] - bf16_hi(h23)));
#pragma unroll
            for (int b = 0; b < D / 16; ++b) o[b] = mfma16k16(vop[b], pl, mfma16k16(vop[b], ph, o[b]));
        }
        wait_vmem<0>();  // every DMA of the wave has landed before the LDS is reused
    }
    if (bad) a.err[0] = 1;
    mfma_decode_finish<D, R>(a, lds_raw, lds_ml, o, m, l, wave, lane, rvalid, item, kvh, hkv, rows);
}

// gfx950 LDS transpose read of bytes: in each group of 16 lanes, lane s gives
// the address of 8 consecutive bytes; lane t = 8a + e receives byte e of the
// chunks of lanes a, a + 2, ..., a + 14 (probed on the device).
__device__ __forceinline__ uint2 lds_read_tr8(const uint8_t *p) {
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    const v2i_t x = __builtin_amdgcn_ds_read_tr8_b64_v2i32((v2i_t __attribute__((address_space(3))) *)(p));
    return __builtin_bit_cast(uint2, x);
}
// Eight int8 values as eight bf16 (exact).
__device__ __forceinline__ uint4 i8x8_to_bf16(uint2 w) {
    const uint2 lo = i8x4_to_bf16(w.x), hi = i8x4_to_bf16(w.y);
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// Split-K decode of int8 PAGED rows on MFMA (up to 8 query rows per kv head
// in an 8-row tile, head_dim 64 / 128): grid, key splits, visibility and
// partial format as decode_mfma_kernel<D, 8>. Each wave streams 32-key tiles
// of its range into an LDS ring of its own (global_load_lds: NSTG stages,
// NSTG tiles in flight while one is computed). A DMA instruction moves whole
// rows (1 KiB: 1024 / D keys), so that every K/V row is fetched by one
// instruction. In LDS a stage holds the tile's K rows and its V rows (key k
// at k * D, its 16-byte unit u at unit u ^ swz(k), swizzles chosen so that
// each operand read below touches every bank at most twice, the minimum for
// 512 bytes) and 256 B of scales (word k the K scale of key k, word 32 + k
// its V scale).
// S^T (16 keys x 16 rows) = K Q^T on v_mfma_f32_16x16x32_bf16, the A operand
// of block kb being keys kperm(kb, i) = 8 (i / 4) + 4 kb + i % 4, K converted
// to bf16 from LDS (exact: int8 has 7 significant bits), scores times the K
// scale; kperm puts lane (col, grp)'s eight scores on keys 8 grp .. 8 grp + 7,
// the layout of the B operand P^T of O^T (16 dims x 16 rows) += V^T P^T on
// v_mfma_f32_16x16x32_bf16 over the tile's 32 keys, whose A operand V^T
// (8 keys of one dim per lane) is one ds_read_b64_tr_b8 per 16 dims. P
// carries the V scale and is split into two bf16 terms. A fused append's new
// rows are quantised as in decode_kernel (by the waves that reach them, into
// LDS; the first of those also stores them).
template <int D>
__global__ __launch_bounds__(256) void decode_i8_mfma_kernel(DecodeArgs a) {
    constexpr int R = 8;                   // rows per tile and partial
    constexpr int T = kI8MfmaKeys;         // keys per tile
    constexpr int NSTG = KVRT_I8_MFMA_STAGES;
    constexpr int KB = T * D;              // K (or V) bytes of a tile
    constexpr int SB = 2 * KB + 256;       // stage: K, V, scales
    constexpr int DPT = 2 * (KB / 1024) + 1;  // DMA instructions per tile
    constexpr int WB = NSTG * SB;          // ring bytes per wave
    constexpr int NQ = kMaxInt8Rows;
    constexpr int kPartBytes = kWaves * R * (D + 4) * 4;
    constexpr int kLdsBytes = kWaves * WB > kPartBytes ? kWaves * WB : kPartBytes;
    constexpr int CPR = D / 16;   // 16-byte units per int8 row
    constexpr int RPI = 64 / CPR;  // rows per DMA instruction
    constexpr int RPB = 256 / D;   // rows per 256 bytes (one pass over the banks)
    static_assert(T == 32 && (D == 64 || D == 128), "int8 MFMA decode tiles");
    static_assert(DPT * NSTG < 64, "outstanding DMAs fit vmcnt");
    static_assert(kLdsBytes + 2 * NQ * D + 8 * NQ + kWaves * (R * 8 + NSTG * 4) <= 80 * 1024,
                  "two workgroups per CU");
    __shared__ __align__(16) uint8_t lds_raw[kLdsBytes];
    __shared__ float2 lds_ml[kWaves * R];
    __shared__ uint32_t lds_unm[kWaves * NSTG];  // per (wave, stage): bit k = key k on an unmapped page
    __shared__ __align__(16) uint4 nrow_k[NQ * CPR], nrow_v[NQ * CPR];
    __shared__ float nrow_s[2 * NQ];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int item = launch_item(a, blockIdx.z);
    const int kvh = blockIdx.y, hkv = gridDim.y;
    const int split = blockIdx.x * kWaves + wave;
    const int slot = a.slots[item];
    const int len = __builtin_amdgcn_readfirstlane(a.len.lens[(int64_t)slot * a.len.stride + a.len.offset]);
    int plen = 0;
    uint32_t pw = ~0u;
    load_prefix(a.pmask, slot, lane, plen, pw);
    const int Qn = a.qn;
    const int rows = a.group * Qn;
    const bool fused = a.k_new != nullptr;
    const int kend = fused ? len + Qn : len;
    const int p0 = kend - Qn;
    const int kstart = a.window > 0 ? max(0, p0 - a.window + 1) : 0;
    const int nk = max(0, kend - kstart);
    int chunk = (nk + a.n_split - 1) / a.n_split;
    chunk = (chunk + T - 1) / T * T;
    const int ws = kstart + split * chunk;
    const int we = min(kend, ws + chunk);
    const int ntiles = we > ws ? (we - ws + T - 1) / T : 0;

    apply_page_edits(a);

    // Q^T as the B operand: column col is row r = col (q head kvh*g + r/Qn,
    // query r % Qn), lane (col, grp) dims 32c + 8grp .. + 7 of step c; rows
    // past the real ones read row 0 and are zeroed
    const int hq = hkv * a.group;
    const bool rvalid = col < rows;
    uint4 qop[D / 32];
    {
        // row col is q head kvh*g + col / Qn, query col % Qn
        const uint16_t *qp = a.q + (((int64_t)item * hq + kvh * a.group) * Qn + (rvalid ? col : 0)) * D + 8 * grp;
#pragma unroll
        for (int c = 0; c < D / 32; ++c) qop[c] = *reinterpret_cast<const uint4 *>(qp + 32 * c);
#pragma unroll
        for (int c = 0; c < D / 32; ++c)
            if (!rvalid) qop[c] = make_uint4(0, 0, 0, 0);
    }
    const int cq = umod_uniform(col, Qn);  // this column's query
    const int hi = rvalid ? p0 + cq : -1;
    const int lo = a.window > 0 ? p0 + cq - a.window + 1 : 0;

    // unit swizzles: K reads take units 2c + g2 of the 16 keys kperm(kb, i),
    // V^T reads unit b of 32 keys
    auto swz_k = [](int k) { return 2 * ((k >> 3) & (CPR / 2 - 1)); };
    auto swz_v = [](int k) { return (k / RPB) & (CPR - 1); };
    // this lane's key (tile-relative) for the row lookup and the scale DMA;
    // the K/V DMAs take their rows from the lanes that looked them up
    const int vkey = lane & 31;
    const float *sc_src = lane < 32 ? a.kv.ks : a.kv.vs;
    // the page-table entries of the wave's first 64 pages, one per lane
    int pwin0 = ws >> a.kv.block_shift;
    int pwin = load_page_window(a.kv, slot, pwin0, lane);
    // q, the page window and the scale source are awaited before the first
    // DMA: the compiler's own wait at a first use inside the loop would count
    // only its own loads and so drain the ring on every tile
#pragma unroll
    for (int c = 0; c < D / 32; ++c) asm volatile("" ::"v"(qop[c].x), "v"(qop[c].y), "v"(qop[c].z), "v"(qop[c].w));
    asm volatile("" ::"v"(pwin), "v"(sc_src));

    const uint32_t ring = lds_addr(lds_raw) + wave * WB;
    const uint8_t *ring_p = lds_raw + wave * WB;
    bool bad = false;  // a visible key on an unmapped page
    // DMA of tile j into stage st. A tile spans at most T pages, so the
    // window, moved to the tile when the tile leaves it, always covers it.
    // Keys past we read key t0's row and are masked; keys on unmapped pages
    // read pool row 0 and are masked (fused new rows excepted: those come
    // from LDS, their page may be mapped by this launch).
    auto dma_tile = [&](int j, int st) __attribute__((always_inline)) {
        const int t0 = ws + j * T;
        if (((min(we, t0 + T) - 1) >> a.kv.block_shift) - pwin0 >= 64) {
            pwin0 = t0 >> a.kv.block_shift;
            pwin = load_page_window(a.kv, slot, pwin0, lane);
            asm volatile("" ::"v"(pwin));  // awaited here, not at a use past the branch
        }
        const int vc = t0 + vkey < we ? t0 + vkey : t0;
        const int vrow = page_row(a.kv, __shfl(pwin, ((vc >> a.kv.block_shift) - pwin0) & 63), kvh, vc);
        const bool unm = t0 + vkey < we && !(fused && t0 + vkey >= len) && vrow < 0;
        bad |= unm;
        const uint32_t bal = (uint32_t)__ballot(unm);
        if (lane == 0) lds_unm[wave * NSTG + st] = bal;
        const int rowc = max(vrow, 0);
        const uint32_t dst = __builtin_amdgcn_readfirstlane(ring + st * SB);
        const int8_t *kb8 = static_cast<const int8_t *>(a.kv.k);
        const int8_t *vb8 = static_cast<const int8_t *>(a.kv.v);
#pragma unroll
        for (int i = 0; i < KB / 1024; ++i) {
            // lane l: unit l % CPR of tile row RPI i + l / CPR, whose pool row
            // the lane of that key looked up
            const int key = RPI * i + lane / CPR;
            const int64_t row = (int64_t)__shfl(rowc, key) * D;
            dma_load16(kb8 + row + 16 * ((lane % CPR) ^ swz_k(key)), dst + i * 1024);
            dma_load16(vb8 + row + 16 * ((lane % CPR) ^ swz_v(key)), dst + KB + i * 1024);
        }
        dma_load4(sc_src + rowc, dst + 2 * KB);
    };

    float m = kNegBig, l = 0.f;  // running max (uniform per column) and this lane's partial sum
    f32x4_t o[D / 16];
#pragma unroll
    for (int b = 0; b < D / 16; ++b) o[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int pro = min(NSTG, ntiles);
    for (int j = 0; j < pro; ++j) dma_tile(j, j);
    // A fused append's new rows, quantised while the first tiles stream in
    // by the waves that reach them, into LDS (the one whose range starts at
    // or before the first of them also stores them; their loads complete
    // after the DMAs issued before them, so the wait for them also covers
    // the first tiles, which the wave computes next)
    if (fused && we > len)
        i8_new_rows<D, NQ, KVRT_LAYOUT_PAGED>(a, item, slot, kvh, hkv, len, Qn, lane, ws <= len, nrow_k, nrow_v,
                                              nrow_s);
    // this lane's K operand keys kperm(kb, col) (dims 32c + 8grp .. + 7 of
    // step c) and V^T source key and half unit
    const int kq0 = 8 * (col >> 2) + (col & 3), kq1 = kq0 + 4;
    const int vk = 8 * grp + ((lane & 15) >> 1);
    auto koff = [&](int k, int c) { return k * D + 16 * ((2 * c + (grp >> 1)) ^ swz_k(k)) + 8 * (grp & 1); };
    const int voff = vk * D + 8 * (lane & 1);
    for (int j = 0; j < ntiles; ++j) {
        const int st = j % NSTG;
        wait_vmem_steps<DPT, NSTG - 1>(min(NSTG - 1, ntiles - 1 - j));
        const int t0 = ws + j * T;
        const uint8_t *kst = ring_p + st * SB, *vst = kst + KB;
        const float *scs = reinterpret_cast<const float *>(kst + 2 * KB);
        uint2 kraw[2][D / 32], vraw[D / 16];
        float ksc[8], vsc[8];
        // a tile that reaches a fused append's new rows (wave-uniform) takes
        // them, quantised, from LDS: per-lane addresses of the K units, V^T
        // sources and scales of those keys point there
        if (fused && t0 + T > len) {
            const uint8_t *nk8 = reinterpret_cast<const uint8_t *>(nrow_k);
            const uint8_t *nv8 = reinterpret_cast<const uint8_t *>(nrow_v);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int kq = kb ? kq1 : kq0;
                const int key = t0 + kq;
                const bool nw = key >= len && key < we;
#pragma unroll
                for (int c = 0; c < D / 32; ++c)
                    kraw[kb][c] = *reinterpret_cast<const uint2 *>(
                        nw ? nk8 + (key - len) * D + 32 * c + 8 * grp : kst + koff(kq, c));
            }
            {
                const int key = t0 + vk;
                const bool nw = key >= len && key < we;
#pragma unroll
                for (int b = 0; b < D / 16; ++b)
                    vraw[b] = lds_read_tr8(nw ? nv8 + (key - len) * D + 16 * b + 8 * (lane & 1)
                                              : vst + voff + 16 * (b ^ swz_v(vk)));
            }
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int key = t0 + 8 * grp + jj;
                const bool nw = key >= len && key < we;
                ksc[jj] = nw ? nrow_s[key - len] : scs[8 * grp + jj];
                vsc[jj] = nw ? nrow_s[NQ + key - len] : scs[32 + 8 * grp + jj];
            }
        } else {
#pragma unroll
            for (int c = 0; c < D / 32; ++c) {
                kraw[0][c] = *reinterpret_cast<const uint2 *>(kst + koff(kq0, c));
                kraw[1][c] = *reinterpret_cast<const uint2 *>(kst + koff(kq1, c));
            }
#pragma unroll
            for (int b = 0; b < D / 16; ++b) vraw[b] = lds_read_tr8(vst + voff + 16 * (b ^ swz_v(vk)));
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                ksc[jj] = scs[8 * grp + jj];
                vsc[jj] = scs[32 + 8 * grp + jj];
            }
        }
        const uint32_t unm = lds_unm[wave * NSTG + st];
        wait_lds();  // the stage is in registers: refill it
        if (j + NSTG < ntiles) dma_tile(j + NSTG, st);
        // S^T for the two 16-key blocks: lane (col, grp) gets keys
        // 8grp + 4kb + v (v < 4) of row col
        f32x4_t s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            s[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < D / 32; ++c) s[kb] = mfma16(i8x8_to_bf16(kraw[kb][c]), qop[c], s[kb]);
        }
        float sc[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int key = t0 + 8 * grp + jj;
            const bool vis = key < we && key <= hi && key >= lo && !((unm >> (8 * grp + jj)) & 1u);
            sc[jj] = vis ? s[jj >> 2][jj & 3] * ksc[jj] * a.scale_log2 : -INFINITY;
        }
        if (t0 < plen) {  // the tile reaches into the prefix mask (wave-uniform)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int key = t0 + 8 * grp + jj;
                sc[jj] = key < plen && !prefix_bit(pw, key) ? -INFINITY : sc[jj];
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) tmax = fmaxf(tmax, sc[jj]);
        tmax = pair<OpMax, 32>(pair<OpMax, 16>(tmax));
        lazy_rescale<D / 16>(tmax, m, l, o);
        float p[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            p[jj] = __builtin_amdgcn_exp2f(sc[jj] - m);
            l += p[jj];
            p[jj] *= vsc[jj];  // dequantise V through P
        }
        // P = P_hi + P_lo in bf16: B operand keys 8grp + jj of row col
        uint32_t ph[4], pl[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ph[i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
            pl[i] = pack_bf16x2(p[2 * i] - bf16_lo(ph[i]), p[2 * i + 1] - bf16_hi(ph[i]));
        }
        const uint4 phv = make_uint4(ph[0], ph[1], ph[2], ph[3]), plv = make_uint4(pl[0], pl[1], pl[2], pl[3]);
#pragma unroll
        for (int b = 0; b < D / 16; ++b) {
            const uint4 va = i8x8_to_bf16(vraw[b]);
            o[b] = mfma16(va, plv, mfma16(va, phv, o[b]));
        }
    }
    wait_vmem<0>();  // every DMA of the wave has landed before the LDS is reused
    if (bad) a.err[0] = 1;
    mfma_decode_finish<D, R>(a, lds_raw, lds_ml, o, m, l, wave, lane, rvalid, item, kvh, hkv, rows);
}

// grid (kv_heads, n_items, chunks), 256 threads: G consecutive threads merge
// one of the R*D outputs of an (item, kv head) from the partials
// decode_kernel wrote; thread j of the G takes partials j, j + G, ... (at most
// 16, all issued at once: one dependent memory round trip). Runs after the
// decode in stream order, so every partial is visible without device-scope
// fences (which on gfx950 write back and invalidate the whole L2 of an XCD).
// Per thread, then across the G lanes in a fixed butterfly (deterministic):
//   M = max m_s, L = sum l_s 2^(m_s - M), out = sum acc_s 2^(m_s - M) / L.
// Chunk 0 of kv head 0 also advances the item's length after a fused append:
// every decode workgroup has read the lengths by then.
template <int D, int R, int G>
__global__ __launch_bounds__(256) void merge_kernel(DecodeArgs a) {
    const int item = blockIdx.y, kvh = blockIdx.x, hkv = gridDim.x;
    const int n_parts = a.n_parts;
    const int Qn = a.qn;
    const int rows = a.group * Qn;
    const int t = blockIdx.z * 256 + threadIdx.x;
    const int idx = t / G, j = t % G;
    const bool live = idx < rows * D;
    const int r = live ? idx / D : 0, d = live ? idx % D : 0;
    const int64_t pbase = ((int64_t)item * hkv + kvh) * a.n_split * R;  // part s, row r at pbase + s*R + r
    const float2 *ml = a.part_ml + pbase + r;
    const float *acc = a.part_acc + (pbase + r) * D + d;
    float M = kNegBig, L = 0.f, O = 0.f;
    merge_partials<G>(j, live ? n_parts : 0, [&](int sp, float2 &m, float &v) {
        m = ml[(int64_t)sp * R];
        v = acc[(int64_t)sp * R * D];
    }, M, L, O);
    if constexpr (G > 1) {
        const float Mg = group_max<G>(M);
        const float w = __builtin_amdgcn_exp2f(M - Mg);
        L = group_sum<G>(L * w);
        O = group_sum<G>(O * w);
    }
    if (live && j == 0) {
        // row r is q head kvh*g + r / Qn, query r % Qn
        a.out[(((int64_t)item * hkv * a.group + kvh * a.group) * Qn + r) * D + d] =
            f32_to_bf16(L > 0.f ? O / L : 0.f);
    }
    if (a.advance && kvh == 0 && blockIdx.z == 0 && threadIdx.x == 0)
        a.len.lens[(int64_t)a.slots[item] * a.len.stride + a.len.offset] += a.qn;
}

// ---------------------------------------------------------------------------
// chunked-prefill attention (MFMA)
// ---------------------------------------------------------------------------
// grid (n_ksplit * kv_heads * g / hw, n_items, ceil(Q / 16)), 64 * NW
// threads with NW = 4 or 8 >= hw: workgroup (x, y, z) serves key range
// x % n_ksplit of the hw q heads kvh*g + (b % (g/hw))*hw + j (wave j < hw,
// b = x / n_ksplit, kvh = b / (g/hw)) of item y over the 16 query rows of
// block ceil(Q / 16) - 1 - z (on the DMA ring with QB = 2: z over ceil(Q / 32)
// pairs of blocks, waves hw .. 2 hw - 1 on the second block of the pair);
// all NW waves stage each 32-key K/V tile into LDS (K row-major, V
// transposed) and the hw computing waves share it. With PF the next tile's
// global loads are issued into registers before the current tile is
// computed, so their latency hides behind the MFMAs. Per tile and computing
// wave:
//   S^T (32 keys x 16 queries) = K Q^T      2 * D/32  v_mfma_f32_16x16x32_bf16
//   online softmax per query column (fp32, exp2 domain)
//   O^T (D x 16) += V^T P^T                 2 * D/16  v_mfma_f32_16x16x32_bf16
// with P split into two bf16 terms for the second product and everything
// accumulated in fp32. MFMA lane layouts (16x16x32): A[row l%16][k 8(l/16)+j],
// B[k 8(l/16)+j][col l%16], D[row 4(l/16)+v][col l%16].

// Key (within a tile) of row i of S^T block b. Chosen so that lane group G
// (lanes 16G..16G+15) ends up with the scores of keys 8G..8G+7 across the two
// blocks, which are exactly the keys of its B operand in V^T P^T.
__device__ __forceinline__ int pf_key(int b, int i) { return 8 * (i >> 2) + 4 * b + (i & 3); }

// Calls f(integral_constant<int, u>) for u = U .. N-1: register arrays
// indexed by u stay in registers.
template <int U, int N>
struct StaticFor {
    template <class F>
    __device__ __forceinline__ static void run(F &&f) {
        if constexpr (U < N) {
            f(std::integral_constant<int, U>{});
            StaticFor<U + 1, N>::run(f);
        }
    }
};

// Tile units: unit c = (row c / (D/8), 16 B segment c % (D/8)) of both the
// K and the V tile, both staged row-major. Keys at or past kend read row
// kclamp (a key of the cache, masked in the softmax).
// Element offset of row kr of the tile at t0 (key t0 + kr; keys at or past
// kend read row kclamp).
template <int D, int LAYOUT>
__device__ __forceinline__ int64_t pf_row_offset(const KVView &kv, int slot, int kvh, int t0, int kclamp, int kend,
                                                 int kr, bool &bad) {
    const int key = t0 + kr;
    if constexpr (LAYOUT == KVRT_LAYOUT_CONTIG) {
        // one multiply-add per row from the (slot, head) base
        const int64_t base = (int64_t)slot * kv.slot_stride + (int64_t)kvh * kv.head_stride;
        return base + (int64_t)(key < kend ? key : kclamp) * D;
    } else if constexpr (LAYOUT == KVRT_LAYOUT_RING) {
        // t0 % rows once per tile: rows of the tile wrap at most once
        const int64_t base = (int64_t)slot * kv.slot_stride + (int64_t)kvh * kv.head_stride;
        const int r0 = t0 % kv.rows, rs = kclamp % kv.rows;
        int rk = r0 + kr;
        rk = rk >= kv.rows ? rk - kv.rows : rk;
        return base + (int64_t)(key < kend ? rk : rs) * D;
    } else {
        const int64_t off = row_offset<LAYOUT>(kv, slot, kvh, key < kend ? key : kclamp, D);
        bad |= off < 0;
        return off < 0 ? 0 : off;
    }
}

template <int D, int LAYOUT, int TK>
__device__ __forceinline__ void pf_fetch_unit(const KVView &kv, int slot, int kvh, int t0, int kclamp, int kend, int c,
                                              u32x4_t &kx, u32x4_t &vx, bool &bad) {
    constexpr int UNITS = TK * (D / 8);
    const uint16_t *kg = static_cast<const uint16_t *>(kv.k);
    const uint16_t *vg = static_cast<const uint16_t *>(kv.v);
    const int cc = c < UNITS ? c : 0;
    const int kr = cc / (D / 8), ks = cc % (D / 8);
    const int64_t off = pf_row_offset<D, LAYOUT>(kv, slot, kvh, t0, kclamp, kend, kr, bad);
    kx = *reinterpret_cast<const u32x4_t *>(kg + off + 8 * ks);
    vx = *reinterpret_cast<const u32x4_t *>(vg + off + 8 * ks);
}

// LDS layout of a staged K or V tile: row r (key) at r * pf_pitch<D>() bf16,
// its 16-B chunk k at chunk position k ^ pf_swz<D>(r). With D >= 128 the
// rows carry 32 B of padding and chunks are XOR-swizzled by bits 3 and 4 of
// the row, so that the 16 rows x 16 B of one S^T A-operand read and the 8 rows
// x 32 B of one V^T transposed read of a half-wave fall on distinct banks
// (64 banks of 4 B); D = 64 keeps 16 B of padding and no swizzle.
template <int D>
constexpr int pf_pitch() { return D >= 128 ? D + 16 : D + 8; }
template <int D>
__device__ __forceinline__ int pf_swz(int r) { return D >= 128 ? (((r >> 3) & 1) * 8) ^ ((r >> 4) & 1) : 0; }
// Chunk swizzle of the unpadded DMA-ring stages (rows of D bf16, 16-B chunk c
// of row r at c ^ pf_rswz(r), r < 32): bits 0, 1, 3 and 4 of the row move
// chunk bits 1, 2, 3 and 0. With 64 banks of 4 B, the 16 rows x 16 B of one
// S^T A-operand read (keys pf_key(b, 0..15)) land on 16 distinct 16-B bank
// groups and the 8 rows x 2 chunks of a half-wave V^T transposed read on 16
// (found by enumerating XOR maps of the row bits); bit 2 is unused, so rows
// r and r + 4 (the two halves of a transposed read) share the swizzle.
__device__ __forceinline__ int pf_rswz(int r) { return ((r & 3) << 1) | (((r >> 3) & 1) << 3) | ((r >> 4) & 1); }

// EXACT: every thread's unit is in the tile (UNITS a multiple of the block),
// so no lane is masked off: a branch here would make the compiler wait for
// every outstanding load at its join, the next tile's prefetch included.
template <int D, int TK, bool EXACT>
__device__ __forceinline__ void pf_stage_unit(uint16_t *sk, uint16_t *sv, int c, const u32x4_t &kx, const u32x4_t &vx) {
    constexpr int UNITS = TK * (D / 8);
    constexpr int KP = pf_pitch<D>();
    if (EXACT || c < UNITS) {
        const int kr = c / (D / 8), ks = (c % (D / 8)) ^ pf_swz<D>(c / (D / 8));
        *reinterpret_cast<u32x4_t *>(&sk[kr * KP + 8 * ks]) = kx;
        *reinterpret_cast<u32x4_t *>(&sv[kr * KP + 8 * ks]) = vx;
    }
}

// A whole tile of TK keys, KU units per thread: unit u of thread t is
// c = t + u * blockDim (the rows of a tile of KS sub-tiles are consecutive).
template <int D, int LAYOUT, int TK, int KU, int NT>
__device__ __forceinline__ void pf_fetch(const KVView &kv, int slot, int kvh, int t0, int kclamp, int kend,
                                         u32x4_t (&kreg)[KU], u32x4_t (&vreg)[KU], bool &bad) {
    StaticFor<0, KU>::run([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        pf_fetch_unit<D, LAYOUT, TK>(kv, slot, kvh, t0, kclamp, kend, threadIdx.x + u * NT, kreg[u], vreg[u], bad);
    });
}

template <int D, int TK, int KU, int NT>
__device__ __forceinline__ void pf_stage(uint16_t *sk, uint16_t *sv, const u32x4_t (&kreg)[KU], const u32x4_t (&vreg)[KU]) {
    constexpr bool EXACT = (TK * (D / 8)) % NT == 0;
    StaticFor<0, KU>::run([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        pf_stage_unit<D, TK, EXACT>(sk, sv, threadIdx.x + u * NT, kreg[u], vreg[u]);
    });
}

template <int D, int LAYOUT, int NW, bool PF, int KS, int G = 0, int QB = 1>
__global__ __launch_bounds__(64 * NW) void prefill_kernel(PrefillArgs a) {
    constexpr int KP = pf_pitch<D>();  // K / V tile row pitch (bf16)
    constexpr int TK = kPfKeys * KS;   // keys per iteration: KS sub-tiles of 32
    constexpr int UNITS = TK * (D / 8);  // 16-B units of a K (or V) tile
    constexpr int KU = (UNITS + 64 * NW - 1) / (64 * NW);  // units per thread
    constexpr int PD = KU <= 2 ? 4 : 2;                      // tiles in flight with PF
    // two K/V tile buffers, so tile t + 1 is staged while tile t is computed
    constexpr int NBUF = 2;
    constexpr int SUB = kPfKeys * KP;   // bf16 elements of one 32-key sub-tile
    constexpr int TILE = KS * SUB;      // bf16 elements of one K (or V) tile buffer
    // G > 0: the LDS DMA ring (bf16 CONTIG / RING, D 128 / 256): NS = KS * G
    // unpadded, swizzled 32-key stages (pf_rswz), G - 1 groups of KS in flight
    constexpr bool RG = G > 0;
    // QB = 2: two consecutive 16-query blocks share the workgroup's staged
    // tiles (half the tile traffic and DMA instructions per block)
    static_assert(QB == 1 || (QB == 2 && RG && D == 128), "query-block pairs: DMA ring, head_dim 128");
    constexpr int NS = KS * (RG ? G : 1);
    constexpr int RSUB = kPfKeys * D;   // bf16 elements of one ring stage (K or V)
    constexpr int LDS_ELEMS = RG ? NS * RSUB : NBUF * TILE;
    static_assert(PF || KS == 1, "the LDS DMA path stages 32-key tiles");
    static_assert(!RG || (PF && (D == 128 || D == 256) && LAYOUT != KVRT_LAYOUT_PAGED && G >= 2 &&
                          (D / 8) % NW == 0), "DMA ring: bf16 CONTIG / RING, D 128 / 256");
    // the KS - 1 upper parts' accumulators fit the tile buffers for the final combine
    static_assert((KS - 1) * (NW / KS) * 16 * D * 4 <= LDS_ELEMS * 2, "part combine fits LDS");
    static_assert((KS - 1) * (NW / KS) * 16 * 8 <= LDS_ELEMS * 2, "part (m, l) fit LDS");
    __shared__ __align__(16) uint16_t sk[LDS_ELEMS];
    __shared__ __align__(16) uint16_t sv[LDS_ELEMS];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int hw = a.heads_per_wg;
    int nhb, rem;
    udivmod_uniform(a.group, hw, nhb, rem);
    // Wave w computes head w % hw over key part (w / hw) % KS of the
    // workgroup's query block w / (hw KS): within every tile, part p takes
    // the 32-key sub-tile p, and the parts' accumulators are combined at the
    // end (KS > 1 puts 2 or 4 waves on one head and query block without
    // staging any tile twice; QB > 1 puts QB blocks on the same tiles).
    int hidx, wrest;
    udivmod_uniform(wave, hw, wrest, hidx);
    const int part = KS > 1 ? wrest % KS : 0;
    const int qsub = QB > 1 ? wrest / KS : 0;  // this wave's block of the workgroup's QB
    // Grid (head part x key range, item, query blocks): workgroups start in
    // linear id order, so the query blocks are the most significant and run
    // last blocks first. Without a window the last blocks see the most keys:
    // the longest workgroups start first and the grid's tail is short ones.
    const int nks = a.n_ksplit;
    int by, ks;
    udivmod_uniform(blockIdx.x, nks, by, ks);
    const int item = blockIdx.y;
    const int qb = gridDim.z - 1 - blockIdx.z;
    int kvh, hb;
    udivmod_uniform(by, nhb, kvh, hb);
    const int hkv = a.kv.kv_heads;
    const int g = a.group, hq = hkv * g;
    const bool computes = wave < hw * KS * QB;
    const int head = kvh * g + hb * hw + (computes ? hidx : 0);
    const int slot = a.slots[item];
    const int L = a.len.lens[(int64_t)slot * a.len.stride + a.len.offset];
    int plen;  // prefix-attention mask of the slot
    uint32_t pw;
    load_prefix(a.pmask, slot, lane, plen, pw);
    const int Qn = a.qn;
    const int qrow0 = (qb * QB + qsub) * 16;   // this wave's block
    const int base_pos = L - Qn;               // position of query row 0
    const int qr = qrow0 + col;                // this lane's query row (S^T / O^T column)
    const bool qvalid = computes && qr < Qn;
    const int pq = base_pos + qr;
    const int lo_q = a.window > 0 ? pq - a.window + 1 : 0;
    // the workgroup's keys: up to its last block's last query, from its first
    // block's first query's window; with a key split, part ks of them in
    // whole tiles
    int kend = base_pos + min(Qn, (qb + 1) * QB * 16);
    int kstart = a.window > 0 ? max(0, base_pos + qb * QB * 16 - a.window + 1) : 0;
    // this wave's own block's keys (QB > 1: a step outside them is skipped)
    const int wkend = base_pos + min(Qn, qrow0 + 16);
    const int wkstart = a.window > 0 ? max(0, base_pos + qrow0 - a.window + 1) : 0;
    const bool wlive = computes && qrow0 < Qn;
    const int kblock = kstart;  // the block's first key: a row of the cache
    if (nks > 1) {
        const int span = (kend - kstart + nks - 1) / nks;
        const int part = (span + kPfKeys - 1) / kPfKeys * kPfKeys;
        const int k0 = kstart + ks * part;
        kend = min(kend, k0 + part);
        kstart = min(k0, kend);
    }
    // Rows fetched past the range read row kclamp and are masked: the range's
    // first key, or the block's first key when the split left this range
    // empty (kstart == kend can be one past the slot's last row, on a page
    // not mapped or, in CONTIG storage, past the layer's rows)
    const int kclamp = kstart < kend ? kstart : kblock;

    // Q^T as the B operand: lane (col, grp) holds d = 32c + 8grp .. +7 of query qr.
    uint4 qop[D / 32];
    {
        const uint16_t *qp = a.q + (((int64_t)item * hq + head) * Qn + (qvalid ? qr : 0)) * D + 8 * grp;
#pragma unroll
        for (int c = 0; c < D / 32; ++c)
            qop[c] = qvalid ? *reinterpret_cast<const uint4 *>(qp + 32 * c) : make_uint4(0, 0, 0, 0);
    }
    float m = kNegBig, l = 0.f;  // running max (uniform per query) and this lane's partial sum
    f32x4_t o[D / 16];
#pragma unroll
    for (int b = 0; b < D / 16; ++b) o[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    bool bad = false;
    // keys this lane's query sees in the block's range: [klo, khi] (none if
    // the lane has no query)
    const int khi = qvalid ? min(kend - 1, pq) : -1;
    const int klo = lo_q;

    // The MFMA work on the tile staged in LDS, keys t0 .. t0 + 31.
    // V^T operand rows through gfx950's LDS transpose read: in each group of
    // 16 lanes, lane s points at key row 8*grp + s/4 (+4 for the second
    // read), dims 4*(s%4) .. +3 of the 16-dim block; lane t = 4a + e then
    // receives dim 4a + e of key rows 8*grp + j, j = 0..3, i.e. A[d][k].
    // (swizzle: row 8grp + ... has bit 3 = grp & 1 and bit 4 = grp >> 1, so
    // chunk (col&3)/2 + 2*b sits at ((col&3)/2 ^ (grp >> 1)) + 2*(b ^ 4*(grp & 1)):
    // blocks b with bit 2 clear read 64 elements further when grp is odd, the
    // others 64 nearer)
    const int vd = D >= 128 ? (grp & 1) * 64 : 0;
    // this wave's sub-tile of every tile buffer (key part `part`)
    const uint16_t *sk_w = sk + part * SUB;
    const uint16_t *sv_base =
        &sv[part * SUB + (8 * grp + (col >> 2)) * KP + 8 * (((col & 3) >> 1) ^ (D >= 128 ? grp >> 1 : 0)) +
            4 * (col & 1)];
    const uint16_t *sv_lo = sv_base + vd, *sv_hi = sv_base - vd;
    auto read_vt = [&](const uint16_t *p) __attribute__((always_inline)) {
        typedef short v4s_t __attribute__((ext_vector_type(4)));
        const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (v4s_t __attribute__((address_space(3))) *)(p));
        const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (v4s_t __attribute__((address_space(3))) *)(p + 4 * KP));
        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
        return make_uint4(l2.x, l2.y, h2.x, h2.y);
    };
    // The work on one staged 32-key tile: kop(b, c) is key row pf_key(b, col)'s
    // A operand of reduction step c, vop(b) the V^T operand of dims 16b ..
    // 16b + 15 (both read from LDS).
    auto tile_core = [&](int t0, auto kop, auto vop) __attribute__((always_inline)) {
        // every key of the tile visible to all 16 queries of the block (the
        // block's first query sees up to its own position, the last one's
        // window starts at or before t0): no per-key mask
        const bool all_visible = qrow0 + 16 <= Qn && t0 + kPfKeys - 1 <= base_pos + qrow0 &&
                                 (a.window == 0 || t0 >= base_pos + qrow0 + 15 - a.window + 1) && t0 >= plen;
        // S^T blocks: rows = keys pf_key(b, i), cols = queries
        f32x4_t s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            s[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            // chunk grp + 4c of key row kr sits at (grp ^ s0) + 4 * (c ^ 2 s3)
            // (s0, s3: bits 4 and 3 of kr): slices c with bit 1 clear read 64
            // elements further when s3 is set, the others 64 nearer
#pragma unroll
            for (int c = 0; c < D / 32; ++c) s[b] = mfma16(kop(b, c), qop[c], s[b]);
        }
        // mask and scale; this lane holds keys 8grp .. 8grp+7 of the tile.
        // Tiles every query sees whole take no per-key test; the others a
        // branch-free one: key in [klo, khi] and passing the prefix mask.
        float sc[8];
        float tmax = -INFINITY;
        if (all_visible) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sc[j] = (j < 4 ? s[0][j] : s[1][j - 4]) * a.scale_log2;
                tmax = fmaxf(tmax, sc[j]);
            }
        } else {
            // bit j of vis8: key k0 + j lies in [klo, khi] and passes the
            // prefix mask; one bit test per key
            const int k0 = t0 + 8 * grp;
            const uint32_t pvis = t0 < plen ? prefix_bits8(pw, k0, plen) : 0xffu;
            const int nhi = min(max(khi - k0 + 1, 0), 8), nlo = min(max(klo - k0, 0), 8);
            const uint32_t vis8 = ((1u << nhi) - 1u) & ~((1u << nlo) - 1u) & pvis;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sc[j] = (vis8 & (1u << j)) != 0 ? (j < 4 ? s[0][j] : s[1][j - 4]) * a.scale_log2 : -INFINITY;
                tmax = fmaxf(tmax, sc[j]);
            }
        }
        tmax = pair<OpMax, 32>(pair<OpMax, 16>(tmax));
        lazy_rescale<D / 16>(tmax, m, l, o);
        // P = P_hi + P_lo, both bf16 (P_lo = the rounding error of P_hi): the
        // two products keep P to ~2^-17 relative, where one bf16 P (2^-9)
        // would be visible in bf16 outputs of few-key rows.
        uint32_t ph[4], pl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float p0 = __builtin_amdgcn_exp2f(sc[2 * j] - m);
            const float p1 = __builtin_amdgcn_exp2f(sc[2 * j + 1] - m);
            l += p0 + p1;
            ph[j] = pack_bf16x2(p0, p1);
            pl[j] = pack_bf16x2(p0 - bf16_lo(ph[j]), p1 - bf16_hi(ph[j]));
        }
        const uint4 pop_hi = make_uint4(ph[0], ph[1], ph[2], ph[3]);
        const uint4 pop_lo = make_uint4(pl[0], pl[1], pl[2], pl[3]);
        // O^T += V^T P^T: A row i = d (16b + col), k = keys 8grp .. +7
#pragma unroll
        for (int b = 0; b < D / 16; ++b) {
            const uint4 va = vop(b);
            o[b] = mfma16(va, pop_lo, mfma16(va, pop_hi, o[b]));
        }
    };
    // the padded, chunk-swizzled tile buffers of the register-staged paths
    auto compute_tile = [&](int t0, auto buf_c) __attribute__((always_inline)) {
        constexpr int BO = decltype(buf_c)::value * TILE;  // the tile's buffer
        tile_core(
            t0,
            [&](int b, int c) __attribute__((always_inline)) {
                // chunk grp + 4c of key row kr sits at (grp ^ s0) + 4 * (c ^ 2 s3)
                // (s0, s3: bits 4 and 3 of kr): slices c with bit 1 clear read 64
                // elements further when s3 is set, the others 64 nearer
                const int kr = pf_key(b, col);
                const int kd = D >= 128 ? ((kr >> 3) & 1) * 64 : 0;
                const uint16_t *kp = &sk_w[BO + kr * KP + 8 * (grp ^ (D >= 128 ? (kr >> 4) & 1 : 0))];
                return *reinterpret_cast<const uint4 *>(kp + 32 * c + ((c >> 1) & 1 ? -kd : kd));
            },
            [&](int b) __attribute__((always_inline)) {
                return read_vt(((b >> 2) & 1 ? sv_hi : sv_lo) + BO + 16 * b);
            });
    };
    // Q is in registers before the first prefetch is issued: inside the loop
    // the compiler then waits only for each tile's own loads, not for the
    // prefetches behind it (vmcnt counts in order).
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    if constexpr (RG) {
        // LDS DMA ring: 32-key tile j (keys kstart + 32 j ..) goes to stage
        // j % NS, K and V rows unpadded and chunk-swizzled (pf_rswz), by
        // global_load_lds_dwordx4 (a 1 KiB row range per instruction, lane l
        // fetching the logical chunk that lands on physical chunk l), the
        // instructions of a tile spread over the waves. Groups of KS tiles
        // are computed one after another (part p takes tile it * KS + p)
        // while the next G - 1 groups are in flight; no registers hold them,
        // and every wait is an explicit vmcnt on this wave's own DMAs (loads
        // complete in issue order) followed by one barrier per group.
        constexpr int RPI = 1024 / (2 * D);   // key rows per DMA instruction
        constexpr int IPT = kPfKeys / RPI;    // instructions per K (or V) tile
        constexpr int DPW = 2 * IPT / NW;     // instructions per wave and tile
        static_assert((2 * IPT) % NW == 0, "a tile's DMAs split evenly over the waves");
        const uint16_t *kg = static_cast<const uint16_t *>(a.kv.k);
        const uint16_t *vg = static_cast<const uint16_t *>(a.kv.v);
        const uint32_t sk_a = lds_addr(sk), sv_a = lds_addr(sv);
        const int ntiles = kend > kstart ? (kend - kstart + kPfKeys - 1) / kPfKeys : 0;
        const int ngroups = (ntiles + KS - 1) / KS;
        const int lrow = lane / (D / 8), pchunk = lane % (D / 8);
        auto issue_tile = [&](int j) __attribute__((always_inline)) {
            const int t0 = kstart + j * kPfKeys;
            const uint32_t stage = (uint32_t)((j % NS) * RSUB) * 2;
#pragma unroll
            for (int i = 0; i < DPW; ++i) {
                const int q = wave + i * NW;      // < IPT: K instruction q, else V instruction q - IPT
                const int ins = q % IPT;
                const int r = ins * RPI + lrow;   // key row of this lane
                const int64_t off = pf_row_offset<D, LAYOUT>(a.kv, slot, kvh, t0, kclamp, kend, r, bad);
                const uint16_t *gp = (q < IPT ? kg : vg) + off + 8 * (pchunk ^ pf_rswz(r));
                const uint32_t dst = (q < IPT ? sk_a : sv_a) + stage + (uint32_t)ins * 1024u;
                dma_load16_cached(gp, __builtin_amdgcn_readfirstlane(dst));
            }
        };
        int issued = min((G - 1) * KS, ntiles);
        for (int j = 0; j < issued; ++j) issue_tile(j);
        // this lane's rows and swizzles in a stage: S^T A operand of key
        // pf_key(b, col) (logical chunk 4c + grp), V^T row 8grp + col/4 (+4)
        // with logical chunk 2b + (col & 3) / 2 and half col & 1
        const int kr0 = pf_key(0, col), kr1 = pf_key(1, col);
        const int ksw0 = grp ^ pf_rswz(kr0), ksw1 = grp ^ pf_rswz(kr1);
        const int rv = 8 * grp + (col >> 2);
        const int vsw = ((col & 3) >> 1) ^ pf_rswz(rv);
        const int voff = rv * D + 4 * (col & 1);
        for (int it = 0; it < ngroups; ++it) {
            // tiles issued after this group's: their DMAs may stay in flight
            const int later = issued - min((it + 1) * KS, ntiles);
            wait_vmem_steps<DPW, (G - 1) * KS>(later);
            __syncthreads();  // every wave's DMAs of group it have landed; group it - 1 is done
            const int next = min((it + G) * KS, ntiles);
            for (int j = issued; j < next; ++j) issue_tile(j);  // into group it - 1's stages
            issued = next;
            const int j = it * KS + part;  // this wave's tile (wave-uniform)
            const int tj = kstart + j * kPfKeys;
            if (wlive && j < ntiles && (QB == 1 || (tj < wkend && tj + kPfKeys > wkstart))) {
                const int sb = (j % NS) * RSUB;
                tile_core(
                    tj,
                    [&](int b, int c) __attribute__((always_inline)) {
                        const int kr = b ? kr1 : kr0, ksw = b ? ksw1 : ksw0;
                        return *reinterpret_cast<const uint4 *>(&sk[sb + kr * D + 8 * ((4 * c) ^ ksw)]);
                    },
                    [&](int b) __attribute__((always_inline)) {
                        typedef short v4s_t __attribute__((ext_vector_type(4)));
                        const uint16_t *p = &sv[sb + voff + 8 * ((2 * b) ^ vsw)];
                        const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (v4s_t __attribute__((address_space(3))) *)(p));
                        const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (v4s_t __attribute__((address_space(3))) *)(p + 4 * D));
                        const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
                        return make_uint4(l2.x, l2.y, h2.x, h2.y);
                    });
            }
        }
    } else if constexpr (PF) {
        // PD tiles in flight in registers (ring slot s holds tiles s, s + PD,
        // ...; keys past kend read row kclamp: in bounds, never visible) and
        // two tile buffers in LDS (tile i in buffer i % 2; PD is even). Per
        // tile one barrier: after it, tile i is staged and every wave is done
        // with tile i - 1, whose buffer then takes tile i + 1 while tile i is
        // computed.
        static_assert(PD % 2 == 0, "tile parity follows the ring slot");
        u32x4_t kreg[PD][KU], vreg[PD][KU];
        StaticFor<0, PD>::run([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            pf_fetch<D, LAYOUT, TK, KU, 64 * NW>(a.kv, slot, kvh, kstart + p * TK, kclamp, kend, kreg[p], vreg[p], bad);
        });
        pf_stage<D, TK, KU, 64 * NW>(sk, sv, kreg[0], vreg[0]);
        pf_fetch<D, LAYOUT, TK, KU, 64 * NW>(a.kv, slot, kvh, kstart + PD * TK, kclamp, kend, kreg[0], vreg[0], bad);
        for (int t0 = kstart; t0 < kend; t0 += PD * TK) {
            StaticFor<0, PD>::run([&](auto pc) {
                constexpr int p = decltype(pc)::value;
                constexpr int pn = (p + 1) % PD;  // ring slot of the next tile
                const int tt = t0 + p * TK;
                if (tt < kend) {
                    __syncthreads();
                    // Staged and refetched unconditionally (past kend the
                    // rows are clamped reads, never computed): a conditional
                    // load here leaves the compiler unsure which loads are
                    // still in flight, and it then waits for all of them
                    // (the next tiles' prefetches included) before staging.
                    pf_stage<D, TK, KU, 64 * NW>(sk + (pn % 2) * TILE, sv + (pn % 2) * TILE, kreg[pn], vreg[pn]);
                    pf_fetch<D, LAYOUT, TK, KU, 64 * NW>(a.kv, slot, kvh, tt + TK + PD * TK, kclamp, kend, kreg[pn],
                                                         vreg[pn], bad);
                    // this wave's 32 keys of the tile (wave-uniform)
                    const int st = tt + part * kPfKeys;
                    if (computes && st < kend) compute_tile(st, std::integral_constant<int, p % 2>{});
                }
            });
        }
    } else {
        // D = 512 (no registers to spare for a prefetch ring): each key row of
        // a tile is one LDS DMA of 64 x 16 B straight into the tile buffer
        // (row pitch and chunk swizzle as pf_stage_unit: lane l fetches the
        // logical chunk that lands on physical chunk l), issued by the waves in
        // turn, one tile ahead, into the other buffer. Per tile: each wave
        // waits for its own DMAs, then one barrier.
        static_assert(D / 8 == 64, "one DMA instruction per key row");
        const uint16_t *kg = static_cast<const uint16_t *>(a.kv.k);
        const uint16_t *vg = static_cast<const uint16_t *>(a.kv.v);
        const uint32_t sk_a = lds_addr(sk), sv_a = lds_addr(sv);
        auto dma_tile = [&](int t0, int buf) __attribute__((always_inline)) {
            for (int rr = wave; rr < 2 * kPfKeys; rr += NW) {  // rr < 32: K row rr, else V row rr - 32
                const int kr = rr % kPfKeys;
                const int64_t off = pf_row_offset<D, LAYOUT>(a.kv, slot, kvh, t0, kclamp, kend, kr, bad);
                const uint16_t *g = (rr < kPfKeys ? kg : vg) + off + 8 * (lane ^ pf_swz<D>(kr));
                const uint32_t dst = (rr < kPfKeys ? sk_a : sv_a) + (uint32_t)(buf * TILE + kr * KP) * 2;
                dma_load16_cached(g, __builtin_amdgcn_readfirstlane(dst));
            }
        };
        if (kstart < kend) dma_tile(kstart, 0);
        for (int t0 = kstart; t0 < kend; t0 += 2 * kPfKeys) {
            StaticFor<0, 2>::run([&](auto pc) {
                constexpr int p = decltype(pc)::value;
                const int tt = t0 + p * kPfKeys;
                if (tt < kend) {
                    wait_vmem<0>();  // this wave's rows of tile tt have landed
                    __syncthreads();  // every wave's have; tile tt - 32's buffer is free
                    if (tt + kPfKeys < kend) dma_tile(tt + kPfKeys, 1 - p);
                    if (computes) compute_tile(tt, std::integral_constant<int, p>{});
                }
            });
        }
    }
    if (bad) a.err[0] = 1;
    l = pair<OpSum, 32>(pair<OpSum, 16>(l));
    if constexpr (KS > 1) {
        // Combine the key parts of each head in a fixed order: parts 1 ..
        // KS - 1 leave (m, l) per query and their o in the drained tile
        // buffers; part 0 rescales everything to the common max and adds.
        __syncthreads();  // every wave is done with the tile buffers
        // o as each lane holds it, [(part - 1) * hw + hidx][block b][lane]: the
        // 64 lanes of a write or read touch 1 KiB of consecutive 16-B chunks (no
        // bank conflicts; a [query][D] layout put the 16 queries of a half-wave
        // D * 4 B apart, on the same banks)
        float4 *xo = reinterpret_cast<float4 *>(sk);
        float2 *xml = reinterpret_cast<float2 *>(sv);  // [((part - 1) * hw + hidx) * QB + qsub][16 queries]
        if (computes && part > 0) {
            const int e = ((part - 1) * hw + hidx) * QB + qsub;
            float4 *dst = xo + (int64_t)e * (D / 16) * 64 + lane;
#pragma unroll
            for (int b = 0; b < D / 16; ++b) dst[64 * b] = make_float4(o[b][0], o[b][1], o[b][2], o[b][3]);
            if (grp == 0) xml[e * 16 + col] = make_float2(m, l);
        }
        __syncthreads();
        if (!computes || part > 0) return;
        float M = m;
#pragma unroll
        for (int q = 1; q < KS; ++q) M = fmaxf(M, xml[(((q - 1) * hw + hidx) * QB + qsub) * 16 + col].x);
        const float w0 = __builtin_amdgcn_exp2f(m - M);
        l *= w0;
#pragma unroll
        for (int b = 0; b < D / 16; ++b) o[b] *= w0;
#pragma unroll
        for (int q = 1; q < KS; ++q) {
            const int e = ((q - 1) * hw + hidx) * QB + qsub;
            const float2 ml = xml[e * 16 + col];
            const float w = __builtin_amdgcn_exp2f(ml.x - M);
            l = fmaf(ml.y, w, l);
            const float4 *src = xo + (int64_t)e * (D / 16) * 64 + lane;
#pragma unroll
            for (int b = 0; b < D / 16; ++b) {
                const float4 x = src[64 * b];
                o[b][0] = fmaf(x.x, w, o[b][0]);
                o[b][1] = fmaf(x.y, w, o[b][1]);
                o[b][2] = fmaf(x.z, w, o[b][2]);
                o[b][3] = fmaf(x.w, w, o[b][3]);
            }
        }
        m = M;
    } else if (!computes) {
        return;
    }
    if (!qvalid) return;
    if (nks > 1) {  // this key range's partial: o unnormalised, (m, l)
        const int64_t pi = (((int64_t)item * hq + head) * Qn + qr) * nks + ks;
        float *po = a.part_o + pi * D + 4 * grp;
#pragma unroll
        for (int b = 0; b < D / 16; ++b)
            *reinterpret_cast<float4 *>(po + 16 * b) = make_float4(o[b][0], o[b][1], o[b][2], o[b][3]);
        if (grp == 0) a.part_ml[pi] = make_float2(m, l);
        return;
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    uint16_t *op = a.out + (((int64_t)item * hq + head) * Qn + qr) * D + 4 * grp;
    // v_cvt_pk_bf16_f32: round to nearest even, as f32_to_bf16 for every
    // non-NaN value, in one instruction per pair
#pragma unroll
    for (int b = 0; b < D / 16; ++b)
        *reinterpret_cast<uint2 *>(op + 16 * b) =
            make_uint2(pack_bf16x2(o[b][0] * inv, o[b][1] * inv), pack_bf16x2(o[b][2] * inv, o[b][3] * inv));
}

// Merge of a key-split prefill: one thread per (item, q head, query) row and
// 4 consecutive dims (16-byte partial loads; D is a power of two, dshift =
// log2(D / 4)), the n_ksplit partials in key order, bf16 out. Per dim the
// arithmetic is merge_partials<1>'s (batches of 16 in partial order).
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a, int D, int dshift, int64_t outs4) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= outs4) return;
    const int64_t row = t >> dshift;  // (item, q head, query)
    const int d = (int)(t & ((1 << dshift) - 1)) * 4;
    const int nks = a.n_ksplit;
    const float2 *ml = a.part_ml + row * nks;
    const float *po = a.part_o + row * nks * D + d;
    constexpr int B = 16;
    float M = kNegBig, L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < nks; s0 += B) {
        float2 m[B];
        float4 v[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int sp = s0 + u;
            m[u] = make_float2(kNegBig, 0.f);
            v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sp < nks) {
                m[u] = ml[sp];
                v[u] = *reinterpret_cast<const float4 *>(po + (int64_t)sp * D);
            }
        }
        float bm = M;
#pragma unroll
        for (int u = 0; u < B; ++u) bm = fmaxf(bm, m[u].x);
        const float c = __builtin_amdgcn_exp2f(M - bm);
        L *= c;
        O.x *= c;
        O.y *= c;
        O.z *= c;
        O.w *= c;
        M = bm;
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const float w = __builtin_amdgcn_exp2f(m[u].x - M);
            L = fmaf(m[u].y, w, L);
            O.x = fmaf(v[u].x, w, O.x);
            O.y = fmaf(v[u].y, w, O.y);
            O.z = fmaf(v[u].z, w, O.z);
            O.w = fmaf(v[u].w, w, O.w);
        }
    }
    const bool any = L > 0.f;
    const uint2 packed = make_uint2(pack_bf16x2(any ? O.x / L : 0.f, any ? O.y / L : 0.f),
                                    pack_bf16x2(any ? O.z / L : 0.f, any ? O.w / L : 0.f));
    *reinterpret_cast<uint2 *>(a.out + row * D + d) = packed;
}

// ---------------------------------------------------------------------------
// small control kernels
// ---------------------------------------------------------------------------
// One workgroup of kPtUpdates threads, thread i edits entry i.
__global__ __launch_bounds__(kPtUpdates) void set_i32_kernel(SetLenArgs a) {
    const int i = threadIdx.x;
    if (a.check) {
        // a rollback validated against host lengths that the device no longer
        // holds (a captured graph advanced it since): refuse it whole
        __shared__ int stale;
        if (i == 0) stale = 0;
        __syncthreads();
        if (i < a.n && a.lens[a.idx[i]] != a.expect[i]) stale = 1;
        __syncthreads();
        if (stale) {
            if (i == 0) a.err[0] = 2;
            return;
        }
    }
    if (i < a.n) a.lens[a.idx[i]] = a.val[i];
}

__global__ __launch_bounds__(256) void copy_rows_kernel(CopyRowsArgs a) {
    const int64_t words = a.row_bytes / 4;
    const int64_t total = a.d0 * a.d1 * a.rows * words;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t w = i % words;
        int64_t t = i / words;
        const int64_t r = t % a.rows;
        t /= a.rows;
        const int64_t b = t % a.d1;
        const int64_t c = t / a.d1;
        const uint32_t x = *reinterpret_cast<const uint32_t *>(a.src + c * a.s0 + b * a.s1 + r * a.sr + 4 * w);
        *reinterpret_cast<uint32_t *>(a.dst + c * a.t0 + b * a.t1 + r * a.tr + 4 * w) = x;
    }
}

// ---------------------------------------------------------------------------
// slot lifecycle: clone / cross-context copy / rollover rebase
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t row_offset_any(const KVView &v, int slot, int head, int pos, int D) {
    if (v.layout == KVRT_LAYOUT_CONTIG) return row_offset<KVRT_LAYOUT_CONTIG>(v, slot, head, pos, D);
    if (v.layout == KVRT_LAYOUT_RING) return row_offset<KVRT_LAYOUT_RING>(v, slot, head, pos, D);
    return row_offset<KVRT_LAYOUT_PAGED>(v, slot, head, pos, D);
}

// grid (chunks, n_entries), 256 threads: every thread step copies 16 B of K
// and of V of one (head, row); int8 layers also copy the row's two scales.
// Source and destination rows must not overlap (different slots).
__global__ __launch_bounds__(256) void slot_copy_kernel(SlotMoveArgs a) {
    const int e = blockIdx.y;
    const LayerDesc S = a.src[a.layer[e]];
    const LayerDesc T = a.dst[a.layer[e]];
    const int D = S.head_dim;
    const int eb = S.dtype == KVRT_INT8 ? 1 : 2;
    const int units = D * eb / 16;
    const int rows = a.rows[e];
    const int64_t total = (int64_t)S.kv.kv_heads * rows * units;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int u = (int)(i % units);
        const int64_t t = i / units;
        const int r = (int)(t % rows);
        const int h = (int)(t / rows);
        const int64_t so = row_offset_any(S.kv, a.src_slot, h, a.src_pos0[e] + r, D);
        const int64_t to = row_offset_any(T.kv, a.dst_slot, h, a.dst_pos0[e] + r, D);
        if (so < 0 || to < 0) {
            a.err[0] = 1;
            continue;
        }
        const int64_t sb = so * eb + u * 16, tb = to * eb + u * 16;
        const uint4 kx = *reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(S.kv.k) + sb);
        const uint4 vx = *reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(S.kv.v) + sb);
        *reinterpret_cast<uint4 *>(static_cast<uint8_t *>(T.kv.k) + tb) = kx;
        *reinterpret_cast<uint4 *>(static_cast<uint8_t *>(T.kv.v) + tb) = vx;
        if (eb == 1 && u == 0) {
            T.kv.ks[to / D] = S.kv.ks[so / D];
            T.kv.vs[to / D] = S.kv.vs[so / D];
        }
    }
}

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float((uint32_t)f32_to_bf16(x) << 16); }

// grid (n_entries, max kv heads), 1024 threads: workgroup (e, h) moves the
// rows[e] <= kMaxRebaseRows rows of kv head h of layer[e] from src_pos0 to
// dst_pos0 within src_slot (bf16 layers). Every thread loads its units (row,
// 8-pair segment: dims [8g, 8g+8) and [D/2 + 8g, D/2 + 8g + 8)) of K and V,
// waits for them, and the workgroup synchronises before the first store, so
// overlapping ranges move correctly. Keys of layers with a RoPE table rotate
// by rope_delta positions: per pair i, with f = fp32(delta * inv_freq[i]),
// c = bf16(cos(f) * scaling), s = bf16(sin(f) * scaling) (cos / sin of the
// fp32 argument rounded from double), x1' = bf16(bf16(x1 c) - bf16(x2 s)),
// x2' = bf16(bf16(x2 c) + bf16(x1 s)).
__global__ __launch_bounds__(1024) void slot_rebase_kernel(SlotMoveArgs a) {
    constexpr int kPer = 4;  // units per thread: 128 rows x 32 segments (D = 512) / 1024
    __shared__ float2 cs[256];
    const int e = blockIdx.x, h = blockIdx.y;
    const LayerDesc L = a.src[a.layer[e]];
    if (h >= L.kv.kv_heads) return;  // the whole workgroup leaves together
    const int D = L.head_dim, half = D / 2;
    const bool rope = L.inv_freq != nullptr;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float c = 1.f, sn = 0.f;
        if (rope) {
            const float f = (float)a.rope_delta * L.inv_freq[i];
            c = bf16_round((float)cos((double)f) * L.rope_scaling);
            sn = bf16_round((float)sin((double)f) * L.rope_scaling);
        }
        cs[i] = make_float2(c, sn);
    }
    const int segs = half / 8;
    const int units = a.rows[e] * segs;
    uint4 k1[kPer], k2[kPer], v1[kPer], v2[kPer];
    int64_t dst[kPer];
    int seg[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int idx = threadIdx.x + j * (int)blockDim.x;
        const bool ok = idx < units;
        const int r = ok ? idx / segs : 0;
        seg[j] = ok ? idx % segs : 0;
        const int64_t so = ok ? row_offset_any(L.kv, a.src_slot, h, a.src_pos0[e] + r, D) : -1;
        const int64_t to = ok ? row_offset_any(L.kv, a.src_slot, h, a.dst_pos0[e] + r, D) : -1;
        if (ok && (so < 0 || to < 0)) a.err[0] = 1;
        dst[j] = (so >= 0 && to >= 0) ? to + 8 * seg[j] : -1;
        k1[j] = k2[j] = v1[j] = v2[j] = make_uint4(0, 0, 0, 0);
        if (dst[j] >= 0) {
            const uint16_t *kp = static_cast<const uint16_t *>(L.kv.k) + so + 8 * seg[j];
            const uint16_t *vp = static_cast<const uint16_t *>(L.kv.v) + so + 8 * seg[j];
            k1[j] = *reinterpret_cast<const uint4 *>(kp);
            k2[j] = *reinterpret_cast<const uint4 *>(kp + half);
            v1[j] = *reinterpret_cast<const uint4 *>(vp);
            v2[j] = *reinterpret_cast<const uint4 *>(vp + half);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // every load of this thread has returned
    __syncthreads();                // ... and of every thread of the workgroup
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        if (dst[j] < 0) continue;
        uint4 n1 = k1[j], n2 = k2[j];
        if (rope) {
            const uint32_t a1[4] = {k1[j].x, k1[j].y, k1[j].z, k1[j].w};
            const uint32_t a2[4] = {k2[j].x, k2[j].y, k2[j].z, k2[j].w};
            uint32_t o1[4], o2[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t lo1 = 0, lo2 = 0;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const float x1 = hh ? bf16_hi(a1[w]) : bf16_lo(a1[w]);
                    const float x2 = hh ? bf16_hi(a2[w]) : bf16_lo(a2[w]);
                    const float2 t = cs[8 * seg[j] + 2 * w + hh];
                    const float y1 = bf16_round(x1 * t.x) - bf16_round(x2 * t.y);
                    const float y2 = bf16_round(x2 * t.x) + bf16_round(x1 * t.y);
                    lo1 |= (uint32_t)f32_to_bf16(y1) << (16 * hh);
                    lo2 |= (uint32_t)f32_to_bf16(y2) << (16 * hh);
                }
                o1[w] = lo1;
                o2[w] = lo2;
            }
            n1 = make_uint4(o1[0], o1[1], o1[2], o1[3]);
            n2 = make_uint4(o2[0], o2[1], o2[2], o2[3]);
        }
        uint16_t *kp = static_cast<uint16_t *>(L.kv.k) + dst[j];
        uint16_t *vp = static_cast<uint16_t *>(L.kv.v) + dst[j];
        *reinterpret_cast<uint4 *>(kp) = n1;
        *reinterpret_cast<uint4 *>(kp + half) = n2;
        *reinterpret_cast<uint4 *>(vp) = v1[j];
        *reinterpret_cast<uint4 *>(vp + half) = v2[j];
    }
}

// grid n_items, 512 threads (8 waves): thread t reads element t of its
// item's mask (t < P; later positions count as visible), and each wave's
// ballot gives mask words 2w and 2w + 1 of the record.
__global__ __launch_bounds__(512) void prefix_pack_kernel(PrefixPackArgs a) {
    const int item = blockIdx.x, t = threadIdx.x;
    bool vis = true;
    if (t < a.plen) {
        const uint8_t *p = a.src + ((int64_t)item * a.item_stride + t) * a.elem_bytes;
        if (a.elem_bytes == 8) vis = *reinterpret_cast<const int64_t *>(p) != 0;
        else if (a.elem_bytes == 4) vis = *reinterpret_cast<const int32_t *>(p) != 0;
        else vis = *p != 0;
    }
    const uint64_t b = __ballot(vis);
    PrefixMask *m = a.dst + a.index[item];
    const int lane = t & 63, wave = t >> 6;
    if (lane == 0) {
        m->bits[2 * wave] = (uint32_t)b;
        m->bits[2 * wave + 1] = (uint32_t)(b >> 32);
    }
    if (t == 0) m->len = a.plen;
}

__global__ __launch_bounds__(256) void zero_kernel(uint4 *p, uint64_t n16) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
         i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
int keys_per_iteration(int head_dim, int rows_tile_, int dtype, int layout) {
    const int vec = dtype == KVRT_INT8 ? 16 : 8;
    const int kpw = 64 / (head_dim / vec);
    return kpw * decode_unroll(rows_tile_, dtype, layout, head_dim);
}

int rows_tile(int rows) {
    if (rows <= 1) return 1;
    if (rows <= 2) return 2;
    if (rows <= 4) return 4;
    if (rows <= 8) return 8;
    if (rows <= 16) return 16;
    return 0;
}

#define KVRT_DISPATCH_D(D_, ...)                       \
    switch (D_) {                                      \
        case 64: { constexpr int HD = 64; __VA_ARGS__; break; }   \
        case 128: { constexpr int HD = 128; __VA_ARGS__; break; } \
        case 256: { constexpr int HD = 256; __VA_ARGS__; break; } \
        case 512: { constexpr int HD = 512; __VA_ARGS__; break; } \
        default: return hipErrorInvalidValue;          \
    }

#define KVRT_DISPATCH_LAYOUT(L_, ...)                                             \
    switch (L_) {                                                                 \
        case KVRT_LAYOUT_CONTIG: { constexpr int LY = KVRT_LAYOUT_CONTIG; __VA_ARGS__; break; } \
        case KVRT_LAYOUT_RING: { constexpr int LY = KVRT_LAYOUT_RING; __VA_ARGS__; break; }     \
        case KVRT_LAYOUT_PAGED: { constexpr int LY = KVRT_LAYOUT_PAGED; __VA_ARGS__; break; }   \
        default: return hipErrorInvalidValue;                                     \
    }

hipError_t launch_append(const AppendArgs &a, int head_dim, int dtype, int grid_x, hipStream_t s) {
    dim3 grid(grid_x, a.n_items), block(256);
    if (dtype == KVRT_INT8) {
        if (a.kv.layout != KVRT_LAYOUT_PAGED) return hipErrorInvalidValue;
        KVRT_DISPATCH_D(head_dim, hipLaunchKernelGGL((append_kernel<HD, KVRT_INT8, KVRT_LAYOUT_PAGED>), grid, block, 0, s, a));
    } else {
        KVRT_DISPATCH_D(head_dim, KVRT_DISPATCH_LAYOUT(a.kv.layout,
            hipLaunchKernelGGL((append_kernel<HD, KVRT_BF16, LY>), grid, block, 0, s, a)));
    }
    return hipGetLastError();
}

hipError_t launch_gather(const GatherArgs &a, int head_dim, int dtype, hipStream_t s) {
    const int rows = head_dim == 64 ? gather_rows<64>() : head_dim == 128 ? gather_rows<128>()
                   : head_dim == 256 ? gather_rows<256>() : gather_rows<512>();
    const int gx = (a.lmax + rows - 1) / rows;
    if (gx < 1 || a.kv.kv_heads < 1 || a.n_items < 1) return hipSuccess;
    dim3 grid(gx, a.kv.kv_heads, a.n_items), block(256);
    if (a.k_new && (dtype != KVRT_BF16 || a.kv.layout == KVRT_LAYOUT_PAGED || !a.v_new || !a.cnt || a.qn < 1))
        return hipErrorInvalidValue;  // the fused append: bf16 CONTIG / RING only
    if (dtype == KVRT_INT8) {
        if (a.kv.layout != KVRT_LAYOUT_PAGED) return hipErrorInvalidValue;
        KVRT_DISPATCH_D(head_dim, hipLaunchKernelGGL((gather_kernel<HD, KVRT_INT8, KVRT_LAYOUT_PAGED>), grid, block, 0, s, a));
    } else {
        KVRT_DISPATCH_D(head_dim, KVRT_DISPATCH_LAYOUT(a.kv.layout,
            hipLaunchKernelGGL((gather_kernel<HD, KVRT_BF16, LY>), grid, block, 0, s, a)));
    }
    return hipGetLastError();
}

// The merge with G threads per output, G the smallest power of two that
// leaves each thread at most 16 partials.
template <int HD, int RT>
static hipError_t launch_merge(const DecodeArgs &a, hipStream_t s) {
    const int parts = a.n_parts;
    const int outs = a.group * a.qn * HD;
    auto go = [&](auto g) {
        constexpr int G = decltype(g)::value;
        const int chunks = (outs * G + 255) / 256;
        hipLaunchKernelGGL((merge_kernel<HD, RT, G>), dim3(a.kv.kv_heads, a.n_items, chunks), dim3(256), 0, s, a);
        return hipGetLastError();
    };
    if (parts <= 16) return go(std::integral_constant<int, 1>{});
    if (parts <= 32) return go(std::integral_constant<int, 2>{});
    if (parts <= 64) return go(std::integral_constant<int, 4>{});
    if (parts <= 128) return go(std::integral_constant<int, 8>{});
    if (parts <= 256) return go(std::integral_constant<int, 16>{});
    return hipErrorInvalidValue;
}

template <int HD, int RT>
static hipError_t launch_decode_rt(const DecodeArgs &a, int dtype, hipStream_t s) {
    if (a.cnt && !decode_wg_merge(HD, RT)) return hipErrorInvalidValue;  // no workgroup partials to merge
    dim3 grid(a.n_split / kWaves, a.kv.kv_heads, a.n_items), block(256);
    if (dtype == KVRT_INT8) {
        // int8 rows carry 16 values per lane: 16 query rows would not fit in registers
        if constexpr (RT > kMaxInt8Rows) return hipErrorInvalidValue;
        else {
            if (a.kv.layout != KVRT_LAYOUT_PAGED) return hipErrorInvalidValue;
            hipLaunchKernelGGL((decode_kernel<HD, RT, KVRT_INT8, KVRT_LAYOUT_PAGED>), grid, block, 0, s, a);
        }
    } else {
        KVRT_DISPATCH_LAYOUT(a.kv.layout,
            hipLaunchKernelGGL((decode_kernel<HD, RT, KVRT_BF16, LY>), grid, block, 0, s, a));
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.cnt) return e;
    return launch_merge<HD, RT>(a, s);
}

// MFMA decode: 16-row tiles, and 8-row tiles for up to 8 rows per kv head;
// int8 rows (PAGED, up to kMaxInt8Rows rows) are converted to bf16 operands.
hipError_t launch_decode_mfma(const DecodeArgs &a, int head_dim, int dtype, int rows_per_head, hipStream_t s) {
    if (a.n_split % kWaves != 0 || a.n_split <= 0 || a.n_parts != a.n_split / kWaves) return hipErrorInvalidValue;
    if (a.pmask && a.kv.layout == KVRT_LAYOUT_PAGED && head_dim >= 512) return hipErrorInvalidValue;  // no mask code
    if (dtype == KVRT_INT8 && (a.kv.layout != KVRT_LAYOUT_PAGED || rows_tile(rows_per_head) > kMaxInt8Rows))
        return hipErrorInvalidValue;
    dim3 grid(a.n_split / kWaves, a.kv.kv_heads, a.n_items), block(256);
    const int rt = rows_tile(rows_per_head);
    if (dtype == KVRT_INT8 && i8_mfma_dma(head_dim, rt)) {
        auto go8 = [&](auto dc) -> hipError_t {
            constexpr int HD = decltype(dc)::value;
            hipLaunchKernelGGL((decode_i8_mfma_kernel<HD>), grid, block, 0, s, a);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess || a.cnt) return e;
            return launch_merge<HD, 8>(a, s);
        };
        return head_dim == 64 ? go8(std::integral_constant<int, 64>{}) : go8(std::integral_constant<int, 128>{});
    }
    auto go = [&](auto rc) -> hipError_t {
        constexpr int RT = decltype(rc)::value;
        KVRT_DISPATCH_D(head_dim, {
            if (dtype == KVRT_INT8) {
                if constexpr (RT <= kMaxInt8Rows)
                    hipLaunchKernelGGL((decode_mfma_kernel<HD, RT, KVRT_LAYOUT_PAGED, KVRT_INT8>), grid, block, 0, s,
                                       a);
            } else {
                KVRT_DISPATCH_LAYOUT(a.kv.layout,
                    hipLaunchKernelGGL((decode_mfma_kernel<HD, RT, LY>), grid, block, 0, s, a));
            }
            hipError_t e = hipGetLastError();
            if (e != hipSuccess || a.cnt) return e;
            return launch_merge<HD, RT>(a, s);
        });
        return hipErrorInvalidValue;
    };
    if (rt >= 1 && rt <= 8) return go(std::integral_constant<int, 8>{});
    if (rt == 16) return go(std::integral_constant<int, 16>{});
    return hipErrorInvalidValue;
}

hipError_t launch_decode(const DecodeArgs &a, int head_dim, int dtype, int rows_per_head, hipStream_t s) {
    if (a.n_split % kWaves != 0 || a.n_split <= 0) return hipErrorInvalidValue;
    const int rt = rows_tile(rows_per_head);
    switch (rt) {
        case 1: KVRT_DISPATCH_D(head_dim, return launch_decode_rt<HD, 1>(a, dtype, s)); break;
        case 2: KVRT_DISPATCH_D(head_dim, return launch_decode_rt<HD, 2>(a, dtype, s)); break;
        case 4: KVRT_DISPATCH_D(head_dim, return launch_decode_rt<HD, 4>(a, dtype, s)); break;
        case 8: KVRT_DISPATCH_D(head_dim, return launch_decode_rt<HD, 8>(a, dtype, s)); break;
        case 16: KVRT_DISPATCH_D(head_dim, return launch_decode_rt<HD, 16>(a, dtype, s)); break;
        default: return hipErrorInvalidValue;
    }
    return hipErrorInvalidValue;
}

template <int HD, int RT>
static hipError_t launch_talker_rt(const TalkerArgs &a, hipStream_t s) {
    if (a.cnt && !decode_wg_merge(HD, RT)) return hipErrorInvalidValue;
    dim3 grid(a.n_split / kWaves, a.kv.kv_heads, a.n_items), block(256);
    hipLaunchKernelGGL((decode_kernel<HD, RT, KVRT_BF16, KVRT_LAYOUT_CONTIG, TalkerArgs>), grid, block, 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.cnt) return e;
    return launch_merge<HD, RT>(a, s);
}

hipError_t launch_decode_talker(const TalkerArgs &a, int head_dim, int rows_per_head, hipStream_t s) {
    if (a.n_split % kWaves != 0 || a.n_split <= 0 || a.kv.layout != KVRT_LAYOUT_CONTIG || a.advance != 0)
        return hipErrorInvalidValue;
    switch (rows_tile(rows_per_head)) {
        case 1: KVRT_DISPATCH_D(head_dim, return launch_talker_rt<HD, 1>(a, s)); break;
        case 2: KVRT_DISPATCH_D(head_dim, return launch_talker_rt<HD, 2>(a, s)); break;
        case 4: KVRT_DISPATCH_D(head_dim, return launch_talker_rt<HD, 4>(a, s)); break;
        case 8: KVRT_DISPATCH_D(head_dim, return launch_talker_rt<HD, 8>(a, s)); break;
        case 16: KVRT_DISPATCH_D(head_dim, return launch_talker_rt<HD, 16>(a, s)); break;
        default: return hipErrorInvalidValue;
    }
    return hipErrorInvalidValue;
}

// The key-split merge: (item, q head, query) rows x D / 4 threads.
hipError_t launch_prefill_merge(const PrefillArgs &a, int head_dim, hipStream_t s) {
    if (head_dim < 4 || (head_dim & (head_dim - 1)) != 0) return hipErrorInvalidValue;
    int dshift = 0;
    while ((1 << dshift) < head_dim / 4) ++dshift;
    const int64_t outs4 = (int64_t)a.n_items * a.kv.kv_heads * a.group * a.qn * (head_dim / 4);
    hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((outs4 + 255) / 256)), dim3(256), 0, s, a, head_dim,
                       dshift, outs4);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs &a, int head_dim, hipStream_t s) {
    const int hw = a.heads_per_wg;
    if (hw <= 0 || a.group % hw != 0 || hw > kPfMaxHeads) return hipErrorInvalidValue;
    if (a.n_ksplit < 1 || (a.n_ksplit > 1 && (!a.part_o || !a.part_ml))) return hipErrorInvalidValue;
    const int ks = a.key_parts;
    if ((ks != 1 && ks != 2 && ks != 4) || ks > prefill_max_parts(head_dim) || hw * ks > 8) return hipErrorInvalidValue;
    if (a.q_blocks != 1 && !(a.q_blocks == 2 && a.ring_groups)) return hipErrorInvalidValue;
    if (a.kv.layout == KVRT_LAYOUT_RING && a.kv.rows < kPfKeys * ks) return hipErrorInvalidValue;  // one wrap per tile
    if (a.ring_groups) {
        // DMA ring: hw * ks * qb waves (at least 2), every one computing
        const int g = a.ring_groups, qbk = a.q_blocks;
        if (!prefill_ring_ok(head_dim, a.kv.layout, ks, g, qbk) || hw * ks * qbk > 8) return hipErrorInvalidValue;
        dim3 grid(a.n_ksplit * a.kv.kv_heads * (a.group / hw), a.n_items, (a.qn + 16 * qbk - 1) / (16 * qbk));
        const int nw = hw * ks * qbk < 2 ? 2 : hw * ks * qbk;
        auto ring = [&](auto d_c, auto ks_c, auto qb_c) -> hipError_t {
            constexpr int HD = decltype(d_c)::value, KS = decltype(ks_c)::value, QB = decltype(qb_c)::value;
            constexpr int G = kPfRingGroups;
            auto go = [&](auto nw_c) {
                constexpr int NW = decltype(nw_c)::value;
                if (a.kv.layout == KVRT_LAYOUT_RING)
                    hipLaunchKernelGGL((prefill_kernel<HD, KVRT_LAYOUT_RING, NW, true, KS, G, QB>), grid,
                                       dim3(64 * NW), 0, s, a);
                else
                    hipLaunchKernelGGL((prefill_kernel<HD, KVRT_LAYOUT_CONTIG, NW, true, KS, G, QB>), grid,
                                       dim3(64 * NW), 0, s, a);
            };
            if (nw == 2) go(std::integral_constant<int, 2>{});
            else if (nw == 4) go(std::integral_constant<int, 4>{});
            else go(std::integral_constant<int, 8>{});
            return hipGetLastError();
        };
        using C128 = std::integral_constant<int, 128>;
        using C256 = std::integral_constant<int, 256>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        hipError_t e;
        if (qbk == 2) e = ks == 1 ? ring(C128{}, I1{}, I2{}) : ring(C128{}, I2{}, I2{});
        else if (head_dim == 256) e = ks == 1 ? ring(C256{}, I1{}, I1{}) : ring(C256{}, I2{}, I1{});
        else e = ks == 1 ? ring(C128{}, I1{}, I1{}) : ring(C128{}, I2{}, I1{});
        if (e != hipSuccess || a.n_ksplit == 1) return e;
        return launch_prefill_merge(a, head_dim, s);
    }
    dim3 grid(a.n_ksplit * a.kv.kv_heads * (a.group / hw), a.n_items, (a.qn + 15) / 16);
    // 4 or 8 waves (hw * ks compute); D = 512 keeps no tile in flight across
    // the MFMAs (registers)
    const bool w8 = hw * ks > 4;
    auto go = [&](auto nw_c, auto ks_c) -> hipError_t {
        constexpr int NW = decltype(nw_c)::value, KS = decltype(ks_c)::value;
        KVRT_DISPATCH_D(head_dim, {
            if constexpr (KS <= prefill_max_parts(HD)) {
                KVRT_DISPATCH_LAYOUT(a.kv.layout, hipLaunchKernelGGL((prefill_kernel<HD, LY, NW, (HD < 512), KS>),
                                                                     grid, dim3(64 * NW), 0, s, a));
                return hipGetLastError();
            } else {
                return hipErrorInvalidValue;
            }
        });
        return hipErrorInvalidValue;
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    using I8 = std::integral_constant<int, 8>;
    hipError_t e;
    if (ks == 1) e = w8 ? go(I8{}, I1{}) : go(I4{}, I1{});
    else if (ks == 2) e = w8 ? go(I8{}, I2{}) : go(I4{}, I2{});
    else e = w8 ? go(I8{}, I4{}) : go(I4{}, I4{});
    if (e != hipSuccess || a.n_ksplit == 1) return e;
    return launch_prefill_merge(a, head_dim, s);
}

hipError_t launch_set_lens(const SetLenArgs &a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(kPtUpdates), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_set_pages(int32_t *pt, int n, const int32_t *idx, const int32_t *val, hipStream_t s) {
    for (int off = 0; off < n; off += kPtUpdates) {
        SetLenArgs a{};
        a.lens = pt;
        a.n = (n - off) < kPtUpdates ? (n - off) : kPtUpdates;
        for (int i = 0; i < a.n; ++i) {
            a.idx[i] = idx[off + i];
            a.val[i] = val[off + i];
        }
        hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(kPtUpdates), 0, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_copy_rows(const CopyRowsArgs &a, hipStream_t s) {
    const int64_t total = a.d0 * a.d1 * a.rows * (a.row_bytes / 4);
    if (total <= 0) return hipSuccess;
    int64_t g = (total + 255) / 256;
    if (g > 8192) g = 8192;
    hipLaunchKernelGGL(copy_rows_kernel, dim3((unsigned)g), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_slot_copy(const SlotMoveArgs &a, int64_t max_units, hipStream_t s) {
    if (a.n_entries <= 0 || max_units <= 0) return hipSuccess;
    if (a.n_entries > kMaxMoveLayers) return hipErrorInvalidValue;
    int64_t g = (max_units + 255) / 256;
    if (g > 2048) g = 2048;
    hipLaunchKernelGGL(slot_copy_kernel, dim3((unsigned)g, a.n_entries), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_slot_rebase(const SlotMoveArgs &a, int max_heads, hipStream_t s) {
    if (a.n_entries <= 0) return hipSuccess;
    if (a.n_entries > kMaxMoveLayers || max_heads <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(slot_rebase_kernel, dim3(a.n_entries, max_heads), dim3(1024), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_prefix_pack(const PrefixPackArgs &a, hipStream_t s) {
    static_assert(kPrefixWords * 32 == 512, "one 512-thread workgroup per mask");
    if (a.n_items <= 0) return hipSuccess;
    if (a.n_items > kMaxItems || a.plen < 0 || a.plen > KVRT_MAX_PREFIX_MASK) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prefix_pack_kernel, dim3(a.n_items), dim3(512), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_zero(void *p, uint64_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    if ((bytes & 15u) != 0 || (reinterpret_cast<uintptr_t>(p) & 15u) != 0) return hipErrorInvalidValue;
    const uint64_t n16 = bytes / 16;
    uint64_t g = (n16 + 255) / 256;
    if (g > 16384) g = 16384;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)g), dim3(256), 0, s, static_cast<uint4 *>(p), n16);
    return hipGetLastError();
}

}  // namespace kvrt

/*
 * mkv.h — C ABI of libmuserve_kv.so, the MI355X (gfx950) KV-cache hot path.
 *
 * Every entry point takes caller-owned device pointers, sizes in elements or
 * bytes, and a hipStream_t passed as `void*` (NULL = the default stream).
 * Nothing here allocates device memory, synchronises, or throws: calls are
 * asynchronous and return an int status (MKV_OK or a negative MKV_E_* code,
 * with a message available from mkv_last_error() on the calling thread).
 *
 * Data-dependent faults that only the device can see (a slot or page id out of
 * range, a sequence longer than its block table) never cause an out-of-bounds
 * access: the kernel skips the offending row (writing zeros where it would
 * have produced output) and ORs an MKV_DEVERR_* bit into the caller-owned
 * int32 `err` word, which the caller reads at its next sync point.
 *
 * Layouts (all row-major, strides in BYTES unless named otherwise):
 *   paged pool  [layers, 2, num_pages, 16, heads, head_dim]   (K plane, V plane)
 *               — the reference layout of muserve/kv_cache.py:4-10,45-49; a
 *               (layer, K|V) plane is an array of `num_pages*16` token rows.
 *   fp8 scales  [layers, 2, num_pages, 16, heads] float32, one per (token, head).
 *   block table [batch, table_width] int32 page ids, seq_lens [batch] int32.
 *
 * The names follow the reference's domain: a "page" is one 16-token block of
 * the pool (muserve/kv_cache.py:77), a "slot" is page*16 + offset.
 */
#ifndef MUSERVE_KV_MKV_H
#define MUSERVE_KV_MKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MKV_ABI_VERSION 1
#define MKV_PAGE_SIZE 16 /* muserve/config.py:36 KV_PAGE_SIZE */

/* host-side status codes */
#define MKV_OK 0
#define MKV_E_INVALID -1   /* bad size / null pointer / negative count       */
#define MKV_E_ALIGN -2     /* pointer or row size not 16-byte aligned        */
#define MKV_E_UNSUPPORTED -3 /* shape outside what the kernels implement     */
#define MKV_E_LAUNCH -4    /* the HIP runtime rejected the launch            */

/* device error bits, OR-ed into the caller's int32 err word */
#define MKV_DEVERR_SLOT 1        /* slot_mapping entry outside [-1, num_slots) */
#define MKV_DEVERR_PAGE 2        /* block-table page id outside [0, num_pages) */
#define MKV_DEVERR_TABLE 4       /* sequence needs more pages than the table holds */
#define MKV_DEVERR_STATE_SLOT 8  /* state-pool slot outside [0, pool_slots)    */
#define MKV_DEVERR_NEW_PAGE 16   /* decode step needed a page but none was given */
#define MKV_DEVERR_BM 32         /* block manager: malformed request or op order */
#define MKV_DEVERR_DUP 64        /* mkv_check_unique: an index appears twice   */

/* ---- meta ------------------------------------------------------------- */

/* ABI version (MKV_ABI_VERSION). No reference counterpart. */
int mkv_version(void);

/* Message of the last non-OK status returned on this thread ("" if none). */
const char* mkv_last_error(void);

/* ---- paged append / gather (bf16 or fp16 rows: plain byte copies) ------- */

/*
 * Slot-mapped append: for every layer l < num_layers and token t < num_tokens
 * with s = slot_mapping[t] >= 0,
 *   K-plane(l)[s] = k_src[l][t],  V-plane(l)[s] = v_src[l][t]
 * where a row is `row_bytes` = heads*head_dim*elem bytes. slot = -1 skips the
 * token; any other slot outside [0, num_slots) sets MKV_DEVERR_SLOT.
 * Slots must be unique within one call (the reference's torch index_put_ with
 * duplicate indices has no defined winner either).
 *
 * Replaces PagedKVCache.write_kv, muserve/kv_cache.py:102-112
 * (cache[l,0,page,slot]=k; cache[l,1,page,slot]=v) with page/slot tensors
 * folded into one int64 slot = page*16 + slot, and the decode-time
 * torch.cat append of muserve/model/qwen35_layer_v2.py:485-492.
 */
int mkv_append_bf16(void* k_pool, void* v_pool, int64_t pool_layer_stride,
                    int64_t num_slots, const void* k_src, const void* v_src,
                    int64_t src_layer_stride, int64_t src_token_stride,
                    const int64_t* slot_mapping, int64_t num_tokens,
                    int32_t num_layers, int32_t row_bytes, int32_t* err,
                    void* stream);

/*
 * Block-table gather into contiguous per-sequence rows. For layer l, sequence
 * b and output row i < out_len, the source position is p = start_b + i
 * (start_b = starts ? starts[b] : 0):
 *   p <  seq_lens[b]:  out(l)[row(b,i)] = plane(l)[block_tables[b][p/16]*16 + p%16]
 *   p >= seq_lens[b]:  padded mode (out_offsets == NULL): row is zero-filled;
 *                      packed mode: row is not written.
 * row(b,i) = b*out_len + i in padded mode ([batch, out_len, row] output, the
 * [B,S,H,D] layout muserve/model/qwen35_model.py:223-249 hands to decode), or
 * out_offsets[b] + i in packed mode (varlen [total, row] output).
 * Output planes of consecutive layers are out_layer_stride bytes apart.
 * Packed mode: out_offsets holds batch + 1 entries, and out_layer_stride is
 * also the capacity of one layer's output (out_layer_stride / row_bytes rows;
 * pass the buffer's size even for one layer). Sequence b's rows are written
 * only inside [out_offsets[b], out_offsets[b+1]) and inside that capacity: a
 * sequence that does not fit (or a negative offset) is cut to the room there
 * is and sets MKV_DEVERR_TABLE.
 *
 * Replaces SequenceKVState.to_page_table_tensor + the contiguous K/V that
 * decode attention reads (muserve/kv_cache.py:149-158,
 * muserve/model/qwen35_layer_v2.py:485-492).
 */
int mkv_gather_bf16(const void* k_pool, const void* v_pool,
                    int64_t pool_layer_stride, int64_t num_pages,
                    const int32_t* block_tables, int64_t table_stride,
                    int32_t table_width, const int32_t* seq_lens,
                    const int32_t* starts, int32_t batch, int64_t out_len,
                    const int64_t* out_offsets, void* k_out, void* v_out,
                    int64_t out_layer_stride, int32_t num_layers,
                    int32_t row_bytes, int32_t* err, void* stream);

/*
 * Decode-step slot assignment for a batch, on the device. For b < batch:
 *   len = seq_lens[b]; if len % 16 == 0 the sequence needs a page:
 *     block_tables[b][len/16] = new_pages[b]   (MKV_DEVERR_NEW_PAGE if < 0)
 *   slot_out[b] = block_tables[b][len/16]*16 + len%16;  seq_lens[b] = len + 1
 * new_pages[b] is the page the host popped for sequence b (-1 when none is
 * needed); the host pops them from the LIFO free list exactly as repeated
 * PagedKVCache.alloc_pages(1) calls would (muserve/kv_cache.py:77-86, the
 * per-token loop of muserve/scripts/test_kv_cache.py:88-92).
 * Replaces SequenceKVState.needs_new_page/current_page/last_page_slot,
 * muserve/kv_cache.py:133-147, for a whole batch in one launch.
 */
int mkv_decode_slots(int32_t* seq_lens, int32_t* block_tables,
                     int64_t table_stride, int32_t table_width,
                     const int32_t* new_pages, int32_t batch,
                     int64_t num_pages, int64_t* slot_out, int32_t* err,
                     void* stream);

/*
 * One batch entry of a scheduler step: `count` new tokens of the request whose
 * persistent block-table row is `row`, at positions [start, start+count).
 * The row holds `held` pages before the step; the step appends `new_pages`
 * pages taken from new_pages[page_off ...]. The entry's tokens occupy
 * [tok_off, tok_off+count) of the step's token arrays.
 */
typedef struct MkvStepEntry {
  int32_t row;
  int32_t start;
  int32_t count;
  int32_t held;
  int32_t new_pages;
  int32_t page_off;
  int32_t tok_off;
  int32_t reserved; /* 0 */
} MkvStepEntry;

/*
 * Scheduler step plan, on the device, for a batch mixing decode tokens and
 * chunked-prefill chunks. For entry i < num_entries (rows unique within a call;
 * token offsets tiling [0, num_tokens) in entry order):
 *   block_tables[row][held + j] = new_pages[page_off + j]      j < new_pages
 *   for t < count, pos = start + t:
 *     pos_out[tok_off + t]  = pos
 *     slot_out[tok_off + t] = page(pos/16)*16 + pos%16
 *   step_tables[i][j] = page j of the row (j < held+new_pages), else 0
 *   step_lens[i] = start + count;  rows_out[i] = row;  cu_seqlens[i] = tok_off
 *   cu_seqlens[num_entries] = num_tokens
 * step_tables may be NULL (no per-step table). An entry whose pages do not
 * cover start+count, whose row or page range is outside the tables, or whose
 * offsets do not tile sets MKV_DEVERR_TABLE and writes slot -1 for its tokens
 * (when its offsets are consistent), length 0, row -1 and a zero step-table
 * row; a page id outside [0, num_pages) sets MKV_DEVERR_PAGE and slot -1.
 * Table strides are in int32 elements.
 *
 * Replaces the per-request SequenceKVState bookkeeping of
 * muserve/kv_cache.py:133-158 (needs_new_page, current_page, last_page_slot,
 * to_page_table_tensor) and the positions/cu_seqlens tensors built per
 * request in muserve/inference_loop.py:100-101,121, for a whole step of the
 * continuous-batching scheduler (muserve/scheduler.py:73-98) with chunked
 * prefill (muserve/config.py:40 CHUNKED_PREFILL_SIZE) in one launch.
 */
int mkv_step_plan(int32_t* block_tables, int64_t table_stride, int32_t table_width,
                  int32_t num_rows, const MkvStepEntry* entries, int32_t num_entries,
                  const int32_t* new_pages, int32_t num_new_pages, int64_t num_pages,
                  int64_t* slot_out, int64_t* pos_out, int64_t num_tokens,
                  int32_t* step_tables, int64_t step_stride, int32_t step_width,
                  int32_t* step_lens, int32_t* rows_out, int64_t* cu_seqlens,
                  int32_t* err, void* stream);

/*
 * Opt-in duplicate check for the index lists the kernels above and below
 * require to be unique (append slot mappings, state-pool scatter / conv /
 * zero slots): every index in [0, limit) of ids[0..n) (int64 when id_bytes
 * is 8, int32 when 4) that appears more than once sets MKV_DEVERR_DUP;
 * indices outside [0, limit), such as the append's -1, are ignored (the
 * consuming kernel flags range faults itself). bitmap is caller-owned device
 * memory of at least ceil(limit / 32) words, zero before the first call; each
 * call leaves it zero again. Calls sharing a bitmap must be ordered (one
 * stream). Issue it before the kernel it guards, on the same stream.
 * No reference counterpart: the reference only requires unique indices
 * (muserve/kv_cache.py:111-112, torch index_put_, whose winner among
 * repeated indices is undefined).
 */
int mkv_check_unique(const void* ids, int32_t id_bytes, int64_t n, int64_t limit,
                     uint32_t* bitmap, int64_t bitmap_words, int32_t* err, void* stream);

/* ---- fp8 e4m3fn quantize-on-append / dequant-gather --------------------- */

/*
 * Append with quantisation: each (token, head) row of head_dim bf16 values x
 * becomes
 *   scale = max(max_i |x_i|, 1e-12f) / 448.0f          (fp32, correctly rounded)
 *   q_i   = e4m3fn_rne(clamp(x_i / scale, -448, 448))   (fp32 divide, RNE)
 * written to the fp8 pool row at the slot, and scale to the scale plane. This
 * is _fast_fp8_quantize(x, block_size=head_dim) of
 * muserve/model/qwen35_layer_v2.py:71-86 applied to K and V separately.
 * head_dim must be 256 (the Qwen3.5 attention head, muserve/config.py:9).
 * Pool strides are in bytes; the scale planes are float arrays with
 * `scale_layer_stride` bytes between layers.
 */
int mkv_append_fp8(void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                   int64_t pool_layer_stride, int64_t scale_layer_stride,
                   int64_t num_slots, const void* k_src, const void* v_src,
                   int64_t src_layer_stride, int64_t src_token_stride,
                   const int64_t* slot_mapping, int64_t num_tokens,
                   int32_t num_layers, int32_t num_heads, int32_t head_dim,
                   int32_t* err, void* stream);

/*
 * Dequant-gather: like mkv_gather_bf16 (same position, padding and packed
 * bounds rules, with bf16 output rows of heads * head_dim * 2 bytes), with
 * each output element bf16_rne(float(q) * scale) for its (token, head) scale.
 * No reference counterpart (the reference keeps no fp8 KV); the formula is
 * the inverse of _fast_fp8_quantize's scaling.
 */
int mkv_gather_dequant_fp8(const void* k_pool, const void* v_pool,
                           const float* k_scale, const float* v_scale,
                           int64_t pool_layer_stride,
                           int64_t scale_layer_stride, int64_t num_pages,
                           const int32_t* block_tables, int64_t table_stride,
                           int32_t table_width, const int32_t* seq_lens,
                           const int32_t* starts, int32_t batch,
                           int64_t out_len, const int64_t* out_offsets,
                           void* k_out, void* v_out, int64_t out_layer_stride,
                           int32_t num_layers, int32_t num_heads,
                           int32_t head_dim, int32_t* err, void* stream);

/* ---- page copies (copy-on-write) ---------------------------------------- */

/*
 * For i < n and every plane q < num_planes:
 *   plane(q)[dst_pages[i]] = plane(q)[src_pages[i]]   (page_bytes each)
 * with plane(q) = pool + q*plane_stride. For the bf16 pool
 * [L,2,P,16,H,D] pass num_planes = 2L, plane_stride = P*page_bytes; for the
 * fp8 scales call again with their own plane geometry. A pair with a negative
 * id is skipped (so mkv_bm_step's cow_src/cow_dst columns can be passed as
 * they are); ids >= num_pages set MKV_DEVERR_PAGE. No reference counterpart: the reference
 * has no copy-on-write; this is the copy a forked sequence needs before its
 * first append into a shared partial page.
 */
int mkv_copy_blocks(void* pool, int64_t plane_stride, int32_t num_planes,
                    int64_t num_pages, int64_t page_bytes,
                    const int32_t* src_pages, const int32_t* dst_pages,
                    int32_t n, int32_t* err, void* stream);

/* ---- GDN recurrent / conv state slot pools ------------------------------ */

/*
 * Slot gather: out[b] = pool[slots[b]] for b < n, each entry `entry_bytes`
 * long, for up to two pools in one launch (pool1 may be NULL, e.g. the
 * [8,128,128] fp32 recurrent state and the [2048,4] bf16 conv state of one
 * GDN layer). Slots outside [0, pool_slots) set MKV_DEVERR_STATE_SLOT and
 * their output is zero-filled. Replaces the per-request state lists the
 * reference threads through forward_decode (muserve/model/qwen35_model.py:
 * 94-126) and the .contiguous() of muserve/inference_loop.py:108.
 */
int mkv_state_gather(const void* pool0, int64_t entry_bytes0, void* out0,
                     const void* pool1, int64_t entry_bytes1, void* out1,
                     int64_t pool_slots, const int32_t* slots, int32_t n,
                     int32_t* err, void* stream);

/* Slot scatter: pool[slots[b]] = in[b]; the inverse of mkv_state_gather.
 * Slots must be unique within one call. */
int mkv_state_scatter(void* pool0, int64_t entry_bytes0, const void* in0,
                      void* pool1, int64_t entry_bytes1, const void* in1,
                      int64_t pool_slots, const int32_t* slots, int32_t n,
                      int32_t* err, void* stream);

/*
 * GDN decode conv in place on the conv-state pool of one layer, one token per
 * request (the decode branch of _gdn_conv1d_apply,
 * muserve/model/qwen35_layer_v2.py:163-201, :187-192):
 *   - conv_pool is [pool_slots, channels, width] bf16: slot s holds the last
 *     `width` inputs of each channel, oldest first (width 3 is the reference's
 *     [C, K-1] state);
 *   - for b < batch, with p = (state[c, width-3 .. width-1], x[b][c]):
 *       out[b][c] = silu(sum_k weight[c][k] * p_k)   (fp32, rounded to bf16)
 *       state[c] <- (state[c, 1 .. width-1], x[b][c])  (slot slots[b])
 *   - x, out are [batch, channels] bf16; weight is [channels, 4] bf16 (the
 *     conv1d.weight [C, 1, 4]).
 * Each request has its own state. The reference's decode instead runs the
 * batch through one state as if it were time, which is the same only at
 * batch 1. Read once and written once per step, the slot needs no dense
 * gather or scatter.
 * Requirements: kernel_size 4, width 3 or 4, channels a multiple of 8,
 * batch <= 65535 (MKV_E_UNSUPPORTED); pointers 16-byte aligned (MKV_E_ALIGN);
 * slots unique. A slot outside [0, pool_slots) gives zeros and sets
 * MKV_DEVERR_STATE_SLOT.
 */
int mkv_gdn_conv_decode(void* conv_pool, int64_t pool_slots, int32_t channels, int32_t width,
                        const int32_t* slots, int32_t batch, const void* x, const void* weight,
                        int32_t kernel_size, void* out, int32_t* err, void* stream);

/*
 * One GDN layer's decode-step state reads in one launch: mkv_state_gather of
 * the batch's recurrent states (state_pool: one layer's [pool_slots,
 * state_bytes] entries -> state_out [batch, state_bytes]) and
 * mkv_gdn_conv_decode on the conv slots (conv_pool [pool_slots, channels,
 * width] -> conv_out [batch, channels]), both indexed by slots. The same
 * results as the two calls, one launch instead of two. Same requirements as
 * each (state_bytes a multiple of 16).
 */
int mkv_gdn_decode_gather(const void* state_pool, int64_t state_bytes, void* state_out,
                          void* conv_pool, int32_t channels, int32_t width, int64_t pool_slots,
                          const int32_t* slots, int32_t batch, const void* x,
                          const void* weight, int32_t kernel_size, void* conv_out,
                          int32_t* err, void* stream);

/* ---- host tier: layered block pack / unpack ------------------------------ */

/*
 * A layered pool holds num_planes planes, plane z starting at
 * pool + z * plane_stride, each an array of pool_blocks blocks of block_bytes.
 * Examples:
 *   - a KV pool [L,2,P,16,H,D]: planes are the L x 2 K|V planes and blocks are
 *     pages (block_bytes = 16*H*D*elem);
 *   - its fp8 scales: 64-byte blocks;
 *   - a GDN state pool: planes are layers and blocks are request slots.
 * Pack copies blocks ids[0..n) of every plane into out, plane-major:
 *   out[(z*n + i)*block_bytes ..] = plane z's block ids[i].
 * Unpack is the inverse (ids unique within a call).
 * out / in may be pinned host memory (hipHostMalloc, torch pin_memory): the
 * kernel then reads or writes it across the host link directly, with no
 * staging copy.
 * Replaces PrefixCache._to_storage / _to_device
 * (muserve/model/prefix_cache.py:36-44: tensor.cpu(), .to(device,
 * non_blocking=True)) for state kept in the library's pools, and caches KV
 * pages, which the reference does not.
 * Requirements (otherwise MKV_E_INVALID / MKV_E_ALIGN):
 *   - pool, out/in, block_bytes and plane_stride are 16-byte aligned;
 *   - plane_stride >= pool_blocks * block_bytes when num_planes > 1;
 *   - 1 <= num_planes <= 65535.
 * An id outside [0, pool_blocks) sets MKV_DEVERR_STATE_SLOT. Pack writes
 * zeros for it; unpack skips it.
 */
int mkv_pack_blocks(const void* pool, int64_t plane_stride, int32_t num_planes,
                    int64_t block_bytes, int64_t pool_blocks, const int32_t* ids, int32_t n,
                    void* out, int32_t* err, void* stream);
int mkv_unpack_blocks(void* pool, int64_t plane_stride, int32_t num_planes,
                      int64_t block_bytes, int64_t pool_blocks, const int32_t* ids, int32_t n,
                      const void* in, int32_t* err, void* stream);

/*
 * Zero-fill of blocks ids[0..n) in every plane of a layered pool (the layout
 * of mkv_pack_blocks): a GDN state pool's planes are its layers and its blocks
 * request slots, so one call gives a newly admitted request zero recurrent
 * (or conv) states in every layer. Replaces the zero initial states the
 * reference builds per request (_init_gdn_states / _init_conv_states,
 * muserve/model/qwen35_model.py:28-49) for slots reused across requests.
 * Requirements as for mkv_pack_blocks; an id outside [0, pool_blocks) sets
 * MKV_DEVERR_STATE_SLOT and is skipped. Ids must be unique within a call.
 */
int mkv_zero_blocks(void* pool, int64_t plane_stride, int32_t num_planes,
                    int64_t block_bytes, int64_t pool_blocks, const int32_t* ids, int32_t n,
                    int32_t* err, void* stream);

/* ---- prefix hashing ------------------------------------------------------ */

/*
 * Per-page prefix hashes. Request r owns the token bytes
 * tokens[tok_offsets[r]*token_bytes, tok_offsets[r+1]*token_bytes); for every
 * full 16-token page i of it,
 *   out[page_offsets[r] + i] = first 8 bytes, big-endian, of
 *                              SHA-256(its first 16*(i+1) tokens)
 * which is int(PrefixCache._hash_tokens(ids[:16*(i+1)]), 16) of
 * muserve/model/prefix_cache.py:31-34 (sha256 of the ids' little-endian
 * bytes, hexdigest()[:16]). token_bytes is 8 (int64 ids) or 4 (int32).
 * page_offsets[r+1]-page_offsets[r] must equal the request's full-page count
 * (floor(tokens/16)); a request where it does not is skipped and sets
 * MKV_DEVERR_TABLE. One lane walks one request's chain, so a launch should
 * carry many requests: a single long prefix is faster on a CPU core.
 */
int mkv_block_hash_sha256(const void* tokens, const int64_t* tok_offsets,
                          const int64_t* page_offsets, int32_t num_requests,
                          int32_t token_bytes, uint64_t* out, int32_t* err,
                          void* stream);

/* ---- block manager (prefix caching, refcounts, copy-on-write, LRU) ------- */

/*
 * Device-resident page bookkeeping for prefix caching. No reference
 * counterpart for the block level: the reference caches whole prefixes
 * (muserve/model/prefix_cache.py:46-105); this keeps its key (the SHA-256
 * prefix hash, here per 16-token page from mkv_block_hash_sha256), its LRU
 * order (OrderedDict move-to-end / popitem(last=False)) and the LIFO free list
 * of muserve/kv_cache.py:77-91, at page granularity.
 *
 * The state is one caller-owned device buffer of mkv_bm_state_bytes(P) bytes
 * (256-byte aligned), initialised by mkv_bm_init with the free stack
 * free_order[0..P) (popped from the end; NULL = 0..P-1). mkv_bm_layout
 * writes 10 int64: table capacity C, ring capacity Q, then the byte offsets of
 * the counters (16 int64: free-stack top, ring head, ring tail, next stamp,
 * evictable pages, tombstones, eviction-log length, then the running totals
 * of admits the many-workgroup passes committed and of admits they covered
 * but left to the one-workgroup tail kernel), the table (C entries of
 * {u64 key, i32 page, i32 copy of the page's refcount}), the page records (P x 32 bytes: i32 refcount, i32
 * flags with bit 0 = cached, u32 LRU stamp, i32 table slot, u64 hash), the
 * free stack (P int32), the LRU ring (Q x u64: page | stamp << 32), the
 * last-occurrence slots (P int32, -1 between steps), the scratch of the
 * many-workgroup passes (4.6 MiB for a release run of up to 2^20 page
 * references: counters, per-op offsets, page ids, bit arrays; plus 8.25 x Q
 * bytes for compacting the ring; plus 26.2 MiB + 8 x P bytes for resolving up
 * to 1024 admits of up to 2048 pages at once: per-admit metadata,
 * per-position probe results, a first-occurrence table of absent hashes,
 * per-page first pinner and late holder, the LRU window and its victims), and
 * the total size.
 *
 * mkv_bm_step runs ops[0..num_ops) with the effect of running them in order
 * (a step of at most 8 ops runs on one workgroup, one op at a time;
 * otherwise a leading run of 1 to 1024 releases is retired by many-workgroup passes;
 * the admits after it, up to 1024 of at most 2048 pages, are resolved
 * together by many-workgroup passes against the state before them, every
 * prediction checked, and the admits before the first one that may differ
 * from the sequential result are committed; one workgroup takes the admits
 * after that in groups of eight, and the rest one op at a time): op r >= 0
 * admits request r, op -(r+1) releases it (r < num_requests, the length of
 * the per-request arrays; hash_offsets has num_requests+1 entries, tables
 * num_requests rows). Request r has num_tokens[r]
 * tokens whose floor(n/16) page hashes are page_hashes[hash_offsets[r] ..
 * hash_offsets[r+1]); they must be prefix keys: two requests' hashes at
 * position i are equal only if their hashes at every position up to i are
 * (a page hash keys the whole prefix up to its page, as the SHA-256 prefix
 * hashes do; hashes of different lengths differ). Admit:
 *   k = number of leading page hashes found in the table;
 *   take = ceil(n/16) - k + (n % 16 != 0); if take > free + evictable - (hits
 *     now evictable): status OOM, nothing changes;
 *   hits: refcount += 1 (leaving the LRU); the other pages come from the free
 *     stack's top, then from evicting the LRU's oldest pages (their hashes
 *     leave the table; each is appended to evict_log while it has room);
 *   pages k.. of the full pages register their hash unless already present;
 *   fork: a child shares every page (refcount += 1); with a partial last page
 *     the child's first append needs a private copy: cow_src/cow_dst[r] name
 *     the pages to copy (mkv_copy_blocks) and child_last[r] the child's page.
 * tables[r][0..ceil(n/16)) receives the parent's page ids, hits[r] = k,
 * status[r] = 0 (admitted), 1 (OOM) or 2 (malformed request: hash count not
 * floor(n/16) or more pages than table_width; sets MKV_DEVERR_BM).
 * Release (child then parent, each from its last page): refcount -= 1; a page
 * reaching 0 goes to the LRU's newest end if cached, else onto the free stack;
 * status[r] becomes 3. Releasing a request that got OOM does nothing;
 * releasing one that is neither admitted nor OOM (never admitted, already
 * released), or an op with r >= num_requests, sets MKV_DEVERR_BM and does
 * nothing.
 */
int64_t mkv_bm_state_bytes(int32_t num_pages);
int mkv_bm_layout(int32_t num_pages, int64_t* out);
int mkv_bm_init(void* state, int32_t num_pages, const int32_t* free_order, void* stream);
int mkv_bm_step(void* state, int32_t num_pages, const int32_t* ops, int32_t num_ops,
                int32_t num_requests, const uint64_t* page_hashes, const int64_t* hash_offsets,
                const int32_t* num_tokens, int32_t* tables, int64_t table_stride,
                int32_t table_width, int32_t* hits, int32_t* child_last,
                int32_t* cow_src, int32_t* cow_dst, int32_t* status,
                int32_t* evict_log, int64_t evict_log_capacity, int32_t* err,
                void* stream);

/*
 * mkv_bm_step in two halves, for a caller that reads results back to the host
 * (no counterpart in the reference). Called with the same arguments, in this
 * order, on one stream, they are mkv_bm_step. _begin launches the release run
 * and the many-workgroup resolution (nothing for a step of at most 8 ops);
 * _end the one-workgroup tail kernel, which runs every op left (none when the
 * counter of committed admits grew by the number of admits in ops). Between the two, the committed admits' tables,
 * hits, status and copy-on-write pairs are final, so a caller may copy them
 * out before _end, whose workgroup needs 96 KiB of LDS and can wait for
 * another kernel's workgroups to leave a CU.
 */
int mkv_bm_step_begin(void* state, int32_t num_pages, const int32_t* ops, int32_t num_ops,
                      int32_t num_requests, const uint64_t* page_hashes,
                      const int64_t* hash_offsets, const int32_t* num_tokens, int32_t* tables,
                      int64_t table_stride, int32_t table_width, int32_t* hits,
                      int32_t* child_last, int32_t* cow_src, int32_t* cow_dst, int32_t* status,
                      int32_t* evict_log, int64_t evict_log_capacity, int32_t* err,
                      void* stream);
int mkv_bm_step_end(void* state, int32_t num_pages, const int32_t* ops, int32_t num_ops,
                    int32_t num_requests, const uint64_t* page_hashes,
                    const int64_t* hash_offsets, const int32_t* num_tokens, int32_t* tables,
                    int64_t table_stride, int32_t table_width, int32_t* hits,
                    int32_t* child_last, int32_t* cow_src, int32_t* cow_dst, int32_t* status,
                    int32_t* evict_log, int64_t evict_log_capacity, int32_t* err,
                    void* stream);

/*
 * Read-only lookup in a block manager's table: for request r < num_requests
 * with page hashes page_hashes[hash_offsets[r] .. hash_offsets[r+1]),
 * pages[i] = the cached page holding hash i (or -1) for every one of them, and
 * hits[r] = the number of leading hashes found — the shared prefix an admit
 * issued now would get. Nothing changes (no LRU touch, no pin). Must not run
 * concurrently with mkv_bm_step on the same state (issue both on one
 * stream). A request with hash_offsets[r+1] < hash_offsets[r] gets hits 0
 * and sets MKV_DEVERR_TABLE. Replaces the scan of PrefixCache.lookup
 * (muserve/model/prefix_cache.py:46-79) without its move_to_end.
 */
int mkv_hash_probe(const void* state, int32_t num_pages, const uint64_t* page_hashes,
                   const int64_t* hash_offsets, int32_t num_requests, int32_t* pages,
                   int32_t* hits, int32_t* err, void* stream);

/* ---- paged decode attention ----------------------------------------------- */

/*
 * Decode attention reading the paged pool directly. For sequence b < batch,
 * with len = seq_lens[b] cached tokens in pages page_table[b][0..ceil(len/16)),
 * and each query head h of KV head kv = h / G (G = num_q_heads / num_kv_heads):
 *   out[b][h] = softmax_j(q[b][h] . k_j * softmax_scale) weighted sum of v_j,
 *   over tokens j < len, k_j / v_j = k_cache / v_cache[page][j % 16][kv].
 * Replaces the paged kernel wrapped by attn_decode (muserve/kernels/attention.py:
 * 29-42: q [B,1,Hq,D], caches [P,16,Hkv,D], cache_seqlens, page_table), i.e.
 * the math of muserve/model/qwen35_layer_v2.py:493-502 without gathering the
 * padded K/V. Scores, softmax and accumulation are fp32; out is bf16 (RNE).
 *   q, out:  [batch, num_q_heads, 256] bf16, contiguous (q[B,1,Hq,D] is too);
 *   k_cache, v_cache: [num_pages, 16, num_kv_heads, 256] bf16 (one layer's
 *            planes of the pool), 16-byte aligned;
 *   page_table: [batch][table_stride] int32, table_width valid columns;
 *   shared_pages: page ids below it may be read by several sequences (a
 *            prefix shared through the block manager, whose page range is
 *            [0, its num_pages)): their K/V are loaded through the caches so
 *            the readers share them; every other page streams past the caches
 *            (non-temporal loads, faster for pages one sequence reads). With
 *            shared_pages > 0, while the pairs (sequence, KV head) number at
 *            most half the kernel's waves, each pair's pages also start a
 *            wave's span, so that the pairs sharing a page read it at the same
 *            time. 0: no page is shared. Results are within the same bound for
 *            every value, bit-identical for every value above 0, and can
 *            differ from those of 0 in the last bits (the pages' split among
 *            the waves, and so the merge order, changes);
 *   max_seq_len: an upper bound of seq_lens; longer sequences are cut to it;
 *   workspace: mkv_decode_attention_workspace_bytes(...) bytes, 16-byte
 *            aligned, contents irrelevant between calls: it receives the
 *            pairs' page prefix and the partial softmax states of pairs cut
 *            between the waves' page spans, which a second kernel merges.
 *            Calls that share a workspace must be ordered (one stream).
 * head_dim must be 256, G one of 1, 2, 4, 8, batch * num_kv_heads at most
 * 4096, max_seq_len at most 2^24 and batch * num_kv_heads * ceil(max_seq_len
 * / 16) below 2^31 (MKV_E_UNSUPPORTED). A page id outside [0, num_pages)
 * skips that page's tokens and sets MKV_DEVERR_PAGE; a length above
 * 16*table_width or max_seq_len is cut to it and sets MKV_DEVERR_TABLE; a
 * sequence of length 0 gets zeros. The workspace size depends on the pair
 * count and G (and the current device's CU count), not on max_seq_len; it
 * returns -1 for an unsupported shape.
 */
int64_t mkv_decode_attention_workspace_bytes(int32_t batch, int32_t num_kv_heads,
                                             int32_t num_q_heads, int32_t max_seq_len);
int mkv_decode_attention_bf16(const void* q, const void* k_cache, const void* v_cache,
                              int64_t num_pages, int64_t shared_pages, int32_t num_kv_heads,
                              int32_t num_q_heads, int32_t head_dim, const int32_t* page_table,
                              int64_t table_stride,
                              int32_t table_width, const int32_t* seq_lens, int32_t batch,
                              int32_t max_seq_len, float softmax_scale, void* out,
                              void* workspace, int64_t workspace_bytes, int32_t* err,
                              void* stream);

/*
 * mkv_decode_attention_bf16 without a workspace argument and without any
 * allocation: the page prefix and partial states live in a file-scope device
 * array of the library (48 MiB, one copy per GPU, held until the process
 * ends), whose address the first call on each device looks up with that
 * device current. No counterpart in the reference: it is for callers that
 * cannot call hipMalloc (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). The caller still passes the inputs, out
 * and err. Limit: mkv_decode_attention_workspace_bytes(...) of the call must
 * fit the array (on MI355X every supported shape needs at most ~17 MB); an
 * unsupported shape or a larger need returns MKV_E_UNSUPPORTED and launches
 * nothing. Calls on one GPU share the array: calls that overlap on one GPU
 * (different streams, or threads without ordering) race and must not be
 * issued; calls ordered on one stream are safe. Results are bit-for-bit
 * those of mkv_decode_attention_bf16 (the same kernels). Same arguments,
 * limits and error bits otherwise.
 */
int mkv_decode_attention_bf16_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                      int64_t num_pages, int32_t num_kv_heads,
                                      int32_t num_q_heads, int32_t head_dim,
                                      const int32_t* page_table, int64_t table_stride,
                                      int32_t table_width, const int32_t* seq_lens,
                                      int32_t batch, int32_t max_seq_len, float softmax_scale,
                                      void* out, int32_t* err, void* stream);

/*
 * The same over an fp16 pool: q, k_cache, v_cache and out are fp16 (scores on
 * the fp16 MFMA, fp32 softmax and accumulation, out rounded to fp16 RNE).
 * fp16 is the reference's default pool dtype (muserve/config.py:37
 * KV_DTYPE = "float16"), and its attn_decode takes q and caches of one dtype
 * (muserve/kernels/attention.py:29-42). Same limits, workspace and error bits
 * as mkv_decode_attention_bf16.
 */
int mkv_decode_attention_f16(const void* q, const void* k_cache, const void* v_cache,
                             int64_t num_pages, int64_t shared_pages, int32_t num_kv_heads,
                             int32_t num_q_heads, int32_t head_dim, const int32_t* page_table,
                             int64_t table_stride,
                             int32_t table_width, const int32_t* seq_lens, int32_t batch,
                             int32_t max_seq_len, float softmax_scale, void* out,
                             void* workspace, int64_t workspace_bytes, int32_t* err,
                             void* stream);

/*
 * The same over an fp8 pool, with the dequantisation fused: k_codes / v_codes
 * are [num_pages, 16, num_kv_heads, 256] e4m3fn codes (16-byte aligned) and
 * k_scales / v_scales the [num_pages, 16, num_kv_heads] fp32 scales that
 * mkv_append_fp8 writes (4-byte aligned). A cached value is code * scale,
 * exact in fp32 (gather_dequant's bf16 rounding is not applied): a token's
 * score is scale_k * (q . codes) and its V weight p * scale_v. Same limits,
 * workspace and error bits as mkv_decode_attention_bf16. Replaces the
 * reference's decode read of the cache (muserve/kernels/attention.py:29-42,
 * muserve/model/qwen35_layer_v2.py:493-502), which has no fp8 pool.
 */
int mkv_decode_attention_fp8(const void* q, const void* k_codes, const void* v_codes,
                             const float* k_scales, const float* v_scales, int64_t num_pages,
                             int64_t shared_pages, int32_t num_kv_heads, int32_t num_q_heads,
                             int32_t head_dim,
                             const int32_t* page_table, int64_t table_stride,
                             int32_t table_width, const int32_t* seq_lens, int32_t batch,
                             int32_t max_seq_len, float softmax_scale, void* out,
                             void* workspace, int64_t workspace_bytes, int32_t* err,
                             void* stream);

/*
 * Decode attention over contiguous per-sequence caches instead of the pool:
 * k_cache / v_cache are [batch, seq_rows, num_kv_heads, 256] (fp16 != 0: fp16,
 * else bf16; q and out of the same type), sequence b attending to its first
 * seq_lens[b] rows. This is attn_decode with page_table None (the reference
 * forwards None to its kernel, muserve/kernels/attention.py:33-42), e.g. over
 * the padded [B, Lpad, H, D] layout mkv_gather_bf16 writes. Rows past
 * seq_rows are never read: lengths above seq_rows (or max_seq_len) are cut
 * and set MKV_DEVERR_TABLE. Same workspace, limits and numerics as
 * mkv_decode_attention_bf16.
 */
int mkv_decode_attention_contig(const void* q, const void* k_cache, const void* v_cache,
                                int32_t fp16, int32_t num_kv_heads, int32_t num_q_heads,
                                int32_t head_dim, int64_t seq_rows, const int32_t* seq_lens,
                                int32_t batch, int32_t max_seq_len, float softmax_scale,
                                void* out, void* workspace, int64_t workspace_bytes,
                                int32_t* err, void* stream);

/* ---- self-test ------------------------------------------------------------ */

/*
 * Varlen prefill attention, causal or not: the math of attn_prefill
 * (muserve/kernels/attention.py:6-25, flash_attn_varlen_func) for 4 query
 * heads per KV head and head_dim 256, bf16 in and out, fp32 softmax and
 * accumulation, probabilities rounded to bf16 for the P V product.
 * Sequence b's queries are rows [cu_seqlens_q[b], cu_seqlens_q[b+1]) of q
 * [num_q_tokens, num_q_heads, 256]; its keys are either
 *   contiguous (page_table NULL): rows [cu_seqlens_k[b], cu_seqlens_k[b+1])
 *     of k/v [kv_units, num_kv_heads, 256], or
 *   paged: the first seq_lens_k[b] tokens of block table row b over a pool
 *     [kv_units pages, 16, num_kv_heads, 256] (chunked prefill: the chunk's
 *     own K/V appended first, so a query also sees the cached prefix).
 * Query t of a sequence with nq queries and nk keys sits at position
 * nk - nq + t (the bottom-right alignment of flash-attention's causal mask)
 * and, when causal, attends to positions 0 .. nk - nq + t; query head h reads
 * KV head h / 4. A query that sees no key gets zeros. max_seqlen_q bounds nq
 * (it sizes the grid). Bad query or key offsets, a sequence longer than its
 * table or than max_seqlen_q set MKV_DEVERR_TABLE; a page id outside the pool
 * sets MKV_DEVERR_PAGE and reads zeros.
 */
int mkv_prefill_attention_bf16(const void* q, const void* k, const void* v, int64_t kv_units,
                               int32_t num_kv_heads, int32_t num_q_heads, int32_t head_dim,
                               const int32_t* page_table, int64_t table_stride,
                               int32_t table_width, const int32_t* cu_seqlens_q,
                               const int32_t* cu_seqlens_k, const int32_t* seq_lens_k,
                               int32_t batch, int64_t num_q_tokens, int32_t max_seqlen_q,
                               float softmax_scale, int32_t causal, int32_t splits,
                               int32_t split_len, void* out, void* workspace,
                               int64_t workspace_bytes, int32_t* err, void* stream);

/*
 * Workspace of mkv_prefill_attention_bf16 with `splits` key ranges (0 for
 * one): with splits > 1 every (query tile, KV head) is cut into ranges of
 * split_len keys (a multiple of 64; the last range runs to the sequence's
 * last key) that separate workgroups attend to, and a second kernel merges
 * their (max, sum, output) per query row and head, writing only the rows of
 * the sequences' queries. That fills the GPU when a step has few, short
 * chunks. With splits > 1 the workspace must be 16-byte aligned and hold
 * these bytes (MKV_E_INVALID otherwise). No reference counterpart.
 */
int64_t mkv_prefill_attention_workspace_bytes(int64_t num_q_tokens, int32_t num_q_heads,
                                              int32_t splits);

/*
 * On-device check of what the fp8 kernels rely on. Adds into counts[7]
 * (device uint64, caller-zeroed): [0] v_cvt_pk_fp8_f32 results that differ
 * from RNE e4m3fn (|x| <= 448, or not NaN for NaN), [1] v_cvt_pk_bf16_f32
 * results that differ from RNE bf16, [2] v_cvt_pk_f32_fp8 decodes that differ
 * from the OCP value, and v_cvt_scalef32_pk_bf16_fp8 (scale 1) decodes that
 * differ from its bf16, [3] fp8 codes where the quantiser's reciprocal divide
 * differs from x / scale, [4] such quotients with |x/scale| >= 2^-12 whose
 * bits differ, [5] fp32 patterns checked (2^32), [6] (absmax, x) pairs
 * checked. Every mismatch count is 0 on a correct gfx950. No reference
 * counterpart: it pins the hardware conversions to torch's CPU semantics.
 */
int mkv_check_conversions(uint64_t* counts, void* stream);

/*
 * Access-pattern probes. Each moves the bytes of one kernel above in the same
 * placement and does nothing else, so that kernel's rate can be set against
 * what its access pattern allows on the device at hand. None has a reference
 * counterpart; they are measurement kernels only.
 *
 * mkv_probe_read_pages: reads the K and V planes (page_bytes 8192 or 4096
 * each, page p at byte p * page_bytes of k_planes / v_planes, num_pages
 * pages) of the n pages listed in pages[n] (int32 on the device; ids outside
 * [0, num_pages) are skipped). walk 0: a workgroup per page; walk 1: the
 * resident grid's waves walk the list, a wave per page, the next page's
 * loads issued before the current one is consumed. nontemporal selects
 * non-temporal or ordinary loads. Nothing is written; sink (16 KiB, 16-byte
 * aligned) keeps the loads alive.
 */
int mkv_probe_read_pages(const void* k_planes, const void* v_planes, int32_t page_bytes,
                         int64_t num_pages, const int32_t* pages, int64_t n, int32_t walk,
                         int32_t nontemporal, void* sink, void* stream);

/*
 * mkv_probe_scatter_pages: for each of `planes` planes y and each listed page
 * x < npages: reads 8 KiB of src at y * src_plane + x * 8192 and writes 4 KiB
 * (the two 16-byte halves of every 32 bytes xor-ed) at y * dst_plane +
 * pages[x] * 4096; ids outside [0, dst_pages) are skipped. The fp8 append's
 * bytes (bf16 rows in, 4 KiB page rows out) without the quantisation.
 */
int mkv_probe_scatter_pages(const void* src, int64_t src_plane, void* dst, int64_t dst_plane,
                            int64_t dst_pages, const int32_t* pages, int32_t npages,
                            int32_t planes, void* stream);

/*
 * mkv_probe_fill: zeros `bytes` (a multiple of 4096) at dst with one 16-byte
 * device-scope non-temporal store a thread, the padded gather's zero tiles.
 */
int mkv_probe_fill(void* dst, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MUSERVE_KV_MKV_H */

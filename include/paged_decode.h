/*
 * paged_decode.h — C ABI of the MI355X (gfx950) paged decode operator.
 *
 * One query token per sequence attends over a paged KV cache:
 *   Q       bf16 [batch, num_heads, head_dim], innermost dim contiguous,
 *           rows 16-byte aligned (strides in elements are multiples of 8)
 *   K, V    bf16 [num_pages, 256, num_kv_heads, head_dim], contiguous (NHD pages)
 *   table   int32 [batch, width] block table, row stride table_stride_b,
 *           width = table_width (1 <= width < 2^22); logical token t of row b
 *           lives in page table[b, t / 256], slot t % 256.  Entries are read
 *           only inside the row's width: a length beyond width * 256 reads
 *           page 0 for the missing entries, never memory outside the table.
 *   lengths int32 [batch], 0 <= lengths[b] <= width * 256
 * Element offset of (page, slot, kv_head, d) is ((page*256+slot)*Hkv+kv_head)*D+d,
 * computed in 64-bit.  Query head h reads kv head h / (num_heads / num_kv_heads).
 *
 * Conventions of every entry point:
 *   - returns PD_OK (0) or a nonzero pd_status; pd_last_error() then holds a
 *     message for the calling thread;
 *   - pointers to tensors are device pointers; nothing is allocated, nothing
 *     synchronizes, no device memory is read on the host, so every launch can
 *     be recorded into a hipGraph on `stream` and replayed with new contents;
 *   - tensor CONTENTS are trusted (live table entries must name valid pages);
 *     use pd_validate_metadata on host copies to check them.
 * `pd_stream_t` is the same type as hipStream_t.
 */
#ifndef PAGED_DECODE_H_
#define PAGED_DECODE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* pd_stream_t;

enum pd_status { PD_OK = 0, PD_EINVAL = 1, PD_ELAUNCH = 2 };

#define PD_PAGE_SIZE 256      /* spec.py:6 */
#define PD_PARTITION_SIZE 1024 /* spec.py:7 */
#define PD_ABI_VERSION 7

/* Split-KV plan; field meanings follow SplitKVPlan (splitkv_plan.py:15-23). */
typedef struct pd_plan {
  int32_t splits;
  int32_t tile_tokens;
  int32_t tokens_per_split;
  int32_t table_capacity_tokens;
  int32_t lse_lanes;
  int32_t sm_count;
  int32_t is_explicit; /* 1 = policy "explicit", 0 = "pinned_geometry" */
} pd_plan;

/* Message describing the last failure on the calling thread ("" if none). */
const char* pd_last_error(void);

/* PD_ABI_VERSION of the built library. */
int pd_abi_version(void);

/* Replaces make_splitkv_plan (splitkv_plan.py:26-56), bit-exact including its
 * float32 rounding points.  max_context_len gives the table capacity through
 * ceil(max_context_len / 256) * 256 (spec.py:36-38).  num_splits = 0 selects
 * the pinned-geometry heuristic, 1..128 an explicit count. */
int pd_make_plan(int32_t max_batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                 int32_t max_context_len, int32_t sm_count, int32_t num_splits, pd_plan* out);

/* Host-memory content check; replaces validate_metadata (reference.py:10-21)
 * as used by validate_device_metadata (runtime.py:38-43): lengths within
 * [0, max_context_len], live pages ceil(len/256) <= width, live entries within
 * [0, num_pages).  `table` and `lengths` are HOST pointers. */
int pd_validate_metadata(const int32_t* table, int64_t table_stride_b, int32_t width,
                         const int32_t* lengths, int32_t batch, int64_t num_pages,
                         int32_t max_context_len);

/* Matched split-KV partition; replaces _normalized_partition
 * (matched_splitkv.py:52-98) as launched by matched_decode (:142-146).
 * Writes partials f32 [batch, num_heads, splits, head_dim] (normalized) and
 * lse f32 [batch, num_heads, splits] (-inf for an empty partition).
 * Partition p covers [p*tokens_per_split, min((p+1)*tokens_per_split, len)),
 * walked in tile_tokens tiles from the last to the first.  Requires
 * head_dim in {64,128,256}, tile_tokens == 16384/head_dim, tokens_per_split a
 * multiple of tile_tokens, num_heads/num_kv_heads <= 16, splits in [1,128].
 * splits * tokens_per_split < 2^31.
 * scale is applied to the scores (exp2 argument uses f32(scale*log2(e))). */
int pd_partition(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                 const void* k, const void* v,
                 const int32_t* table, int64_t table_stride_b, int32_t table_width,
                 const int32_t* lengths,
                 float* partials, float* lse,
                 int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                 int32_t splits, int32_t tokens_per_split, int32_t tile_tokens,
                 double scale, pd_stream_t stream);

/* Stable LSE merge; replaces _lse_merge (matched_splitkv.py:101-127) as
 * launched by matched_decode (:147-149).  Writes out bf16 [batch, num_heads,
 * head_dim].  lse_lanes is the plan's lane count, a power of two in [1, 64]
 * no larger than the next power of two of splits.  It sets the float32
 * summation order of the log-sum, as in the reference: lane j sums splits
 * j, j + lse_lanes, ... in order, then a halving tree adds the lanes. */
int pd_lse_merge(const float* partials, const float* lse, void* out,
                 int32_t batch, int32_t num_heads, int32_t head_dim, int32_t splits,
                 int32_t lse_lanes, pd_stream_t stream);

/* int32 counters per (sequence, kv head) in pd_matched_decode's `counters`. */
#define PD_FUSED_COUNTERS_PER_GROUP 128

/* Matched split-KV decode: the partition of pd_partition plus the LSE merge of
 * pd_lse_merge, bit-identical to pd_partition followed by pd_lse_merge.
 * Replaces the two launches of matched_decode (matched_splitkv.py:142-149).
 * Writes partials, lse and out bf16 [batch, num_heads, head_dim].  The merge
 * sums with the plan's lse_lanes, min(next_pow2(splits), 32 if
 * head_dim % 128 == 0 else 16).
 * With `counters` (non-NULL) it is one fused launch.  With splits of one tile
 * (tokens_per_split == tile_tokens) the merge of each GQA group is shared by
 * the last wavefront to finish each quarter of the head_dim columns;
 * otherwise the last workgroup of each (sequence, kv head) merges the whole
 * group.  `counters` is int32 [batch * num_kv_heads *
 * PD_FUSED_COUNTERS_PER_GROUP] (four counters per group, each on a 128-byte
 * line), all zero before the first call; every completed call leaves it all
 * zero again, so the launch can be replayed from a graph without a reset.
 * Calls that share `counters` must not run concurrently.  The partials are
 * published with device-scope stores and read with device-scope loads, so the
 * merge may run on any XCD.
 * With counters NULL it runs the partition and the merge as two launches,
 * except for a plan of one split of more than one tile (splits == 1,
 * tokens_per_split > tile_tokens): the merge of one split weighs it by exactly
 * 1, so the partition writes out = bf16(partial) itself (-0 as +0, 0 for an
 * empty sequence) and nothing else is launched. */
int pd_matched_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                      const void* k, const void* v,
                      const int32_t* table, int64_t table_stride_b, int32_t table_width,
                      const int32_t* lengths,
                      float* partials, float* lse, int32_t* counters, void* out,
                      int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                      int32_t splits, int32_t tokens_per_split, int32_t tile_tokens,
                      double scale, pd_stream_t stream);

/* Bytes of the static device scratch of pd_matched_decode_noalloc. */
#define PD_NOALLOC_SCRATCH_BYTES (16 << 20)

/* Allocation-free matched split-KV decode.  This entry point has no
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory or pass a workspace (code under hipGraph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, output and
 * results (bit for bit) as pd_matched_decode without its partials, lse and
 * counters: the split workspace lives in a static device array of
 * PD_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, so
 * batch * num_heads * splits * (head_dim + 1) * 4 bytes (plus 256 for
 * alignment) must fit in it, or PD_EINVAL is returned.  It calls no
 * hipMalloc, hipFree or allocating library routine.  Every call on one GPU
 * shares that GPU's scratch, so calls that overlap on one GPU (two streams,
 * two threads) race; calls ordered on one stream do not. */
int pd_matched_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                              const void* k, const void* v,
                              const int32_t* table, int64_t table_stride_b, int32_t table_width,
                              const int32_t* lengths, void* out,
                              int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t splits, int32_t tokens_per_split,
                              int32_t tile_tokens, double scale, pd_stream_t stream);

/* Base decode: FP32 online softmax over the whole context with FP32
 * probabilities, out = acc / denom (0 for an empty row), for every query head.
 * One workgroup per (kv head, sequence) serves the kv head's query heads (16 at
 * a time), so K/V is read once per kv head; at head_dim 64, one workgroup
 * serves four adjacent kv heads when num_kv_heads is a multiple of 4 and they
 * have at most 4 query heads each, else two when num_kv_heads is even and they
 * have at most 8 (a token's rows of those heads are one contiguous read).
 * Replaces _base (kernels.py:10-41) as launched by paged_decode
 * (runtime.py:109).  Writes out rows [0, batch). */
int pd_base(const void* q, int64_t q_stride_b, int64_t q_stride_h,
            const void* k, const void* v,
            const int32_t* table, int64_t table_stride_b, int32_t table_width,
            const int32_t* lengths,
            void* out, int32_t batch, int32_t num_heads, int32_t num_kv_heads,
            int32_t head_dim, double scale, pd_stream_t stream);

/* Fixed-size split-K partition: unnormalized (m, l, acc) per partition of
 * partition_size tokens, m in scaled units, every partition written (empty ones
 * as m = -inf, l = 0, acc = 0).  When the device has at least as many CUs as
 * pd_base has workgroups (one per kv head group and sequence), those
 * workgroups each walk their sequence's context and write every partition as
 * they pass it; with fewer, one workgroup runs per partition, as in the
 * reference's grid.  Both write the same bits.  Replaces _split
 * (kernels.py:44-80) as launched by paged_decode (runtime.py:111-113).
 * maxima/denoms f32 [batch, num_heads, partitions], accums f32 [batch,
 * num_heads, partitions, D] (16-byte aligned); the row stride of all three is
 * `partitions`; partition_size a positive multiple of 16384 / head_dim;
 * partitions * partition_size < 2^31. */
int pd_split_fixed(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                   const void* k, const void* v,
                   const int32_t* table, int64_t table_stride_b, int32_t table_width,
                   const int32_t* lengths,
                   float* maxima, float* denoms, float* accums,
                   int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                   int32_t partitions, int32_t partition_size, double scale,
                   pd_stream_t stream);

/* m/l/acc merge; replaces _merge (kernels.py:83-100) as launched by
 * paged_decode (runtime.py:114-116): M = max m_p (-inf -> 0), f_p =
 * exp(m_p - M), out = sum f_p acc_p / sum f_p l_p (a zero total divides by
 * 1), the sums in partition order.  Writes out rows [0, batch). */
int pd_ml_merge(const float* maxima, const float* denoms, const float* accums, void* out,
                int32_t batch, int32_t num_heads, int32_t head_dim, int32_t partitions,
                pd_stream_t stream);

/* The reference's fixed-split backend in one call (_split + _merge,
 * runtime.py:111-116): the workspace as pd_split_fixed writes it, and the
 * merged output in out.  When the walks fill the device, the walking
 * workgroups merge their sequence's partitions as they complete them (from
 * the last to the first, with a running maximum: the same formula as
 * pd_ml_merge in another order and float32 rounding) and write out directly,
 * in one launch; otherwise one workgroup runs per partition and a merge
 * kernel with the walk's order and arithmetic follows.  Both grids write the
 * same workspace and output bits. */
int pd_split_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                    const void* k, const void* v,
                    const int32_t* table, int64_t table_stride_b, int32_t table_width,
                    const int32_t* lengths,
                    float* maxima, float* denoms, float* accums, void* out,
                    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                    int32_t partitions, int32_t partition_size, double scale,
                    pd_stream_t stream);

/* Small-batch split of the base and fixed-split protocols; no counterpart in
 * the reference, whose _base and _split grids already spread a sequence over
 * (query heads[, partitions]) programs (runtime.py:109-113).  pd_base and
 * pd_split_fixed walk each sequence in one workgroup per kv head group, so a
 * batch of fewer walks than half of sm_count leaves CUs idle; the walks are
 * counted for `batch` rounded up to a power of two.  For such a batch this
 * returns a cut of a table of `table_width` pages into *chunks >= 2 partitions
 * of *chunk_tokens tokens (a multiple of 16384 / head_dim; about sm_count /
 * walks of them, at most 128): run pd_split_fixed(partitions, partition_size =
 * *chunk_tokens) and pd_ml_merge over partitions = ceil(w * 256 /
 * *chunk_tokens) for a call whose table has w <= table_width pages.  That
 * computes the same attention as pd_base or the 1024-token pd_split_fixed with
 * other float32 rounding.  Partitions past a sequence's length are empty and
 * leave the merge's bits unchanged, and each sequence's partitions are its own,
 * so a sequence's output does not depend on w, on the other sequences, or on
 * empty sequences padding the batch below its next power of two (a graph
 * bucket), as long as table_width is the same.  Otherwise *chunks = 1 and
 * *chunk_tokens = table_width * 256: run the backend itself.  Host only. */
int pd_plan_chunks(int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                   int32_t table_width, int32_t sm_count, int32_t* chunks,
                   int32_t* chunk_tokens);

/* Size of a chunk workspace for pd_plan_chunks (no counterpart in the
 * reference): *rows = the largest batch * num_heads * chunks it returns for any
 * batch <= max_batch and any table width (0 if none is cut), so maxima and
 * denoms of *rows floats and accums of *rows * head_dim floats serve every
 * call (batch <= max_batch, any w).  Host only. */
int pd_chunk_rows(int32_t max_batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                  int32_t sm_count, int64_t* rows);

/* KV-cache write of token rows through a flat slot mapping; replaces the
 * store_kvcache Triton kernel of the nano-vLLM overlay
 * (overlays/nano-vllm/nanovllm/layers/attention.py:10-38).  For token i with
 * slot = slot_mapping[i] >= 0, copies row_elems (= num_kv_heads * head_dim)
 * bf16 of key + i*key_stride to k_cache + slot*row_elems, and the same for
 * value/v_cache; slot -1 (a padded graph entry) is skipped.  Rows, caches and
 * strides must be 16-byte aligned (strides multiples of 8 elements, at least
 * row_elems).  Contents are trusted: slots must lie inside the caches. */
int pd_store_kv(const void* key, int64_t key_stride, const void* value, int64_t value_stride,
                void* k_cache, void* v_cache, const int32_t* slot_mapping, int64_t num_tokens,
                int32_t row_elems, pd_stream_t stream);

/* KV-cache write of a [batch, num_kv_heads, steps, head_dim] chunk into
 * 256-slot pages; replaces the index_copy_ of PagedHybridCache.update
 * (src/paged_decode/hybrid.py:63-72).  Element (b, h, s, d) goes to page
 * table[b, positions[s] / 256], slot positions[s] % 256, kv head h.  `positions`
 * is int64 [steps]; k_pages and v_pages hold num_pages pages each.  A negative
 * position, a page index at or past table_width, or a table entry outside
 * [0, num_pages) skips the row (the reference's index_copy_ rejects such an
 * index; here nothing is written outside the pool).  head_dim in
 * {64, 128, 256}; strides in elements, multiples of 8; pointers 16-byte
 * aligned. */
int pd_store_kv_pages(const void* key, int64_t key_stride_b, int64_t key_stride_h,
                      int64_t key_stride_s, const void* value, int64_t value_stride_b,
                      int64_t value_stride_h, int64_t value_stride_s, void* k_pages,
                      void* v_pages, int64_t num_pages, const int32_t* table,
                      int64_t table_stride_b,
                      int32_t table_width, const int64_t* positions, int32_t batch,
                      int32_t num_kv_heads, int32_t steps, int32_t head_dim, pd_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGED_DECODE_H_ */

// Paged decode attention kernels for MI355X (gfx950, CDNA4) and their C-ABI
// launchers.  See include/paged_decode.h for the tensor contract.
//
// Kernels
//   cols_loader        one 512-thread workgroup per (split, kv head, sequence)
//                      (per (kv head, sequence) for the base and fixed-split
//                      protocols, which walk the whole context, and per run
//                      of consecutive short splits for the matched walk):
//                      QK^T on MFMA (v_mfma_f32_16x16x32_bf16), FP32 online
//                      softmax over 16384/D-row tiles walked last-to-first, P
//                      through LDS and PV on MFMA split across the four
//                      compute wavefronts by output columns, while four loader
//                      wavefronts copy the K and V rows of the next tiles into
//                      LDS (buffer_load ... lds) and store completed
//                      partitions of the walks.  Three protocols: matched
//                      (bf16 p, normalized FP32 partial + LSE), base (FP32 p,
//                      whole context, bf16 out) and fixed split (FP32 p,
//                      (m, l, acc) per partition, optionally merged in the
//                      kernel).  D = 64, 128 and 256.
//   matched_tile       the matched protocol for splits of exactly one tile,
//                      with PV split across the wavefronts by output columns.
//   lse_merge          one wavefront per (sequence, query head, 64 columns):
//                      stable log-sum-exp merge of the split partials, bf16 out.
//   ml_merge           one wavefront per (sequence, query head, 64 columns):
//                      merge of the (m, l, acc) states in the reference's
//                      order; ml_online_merge the same in the fixed-split
//                      walk's order (running maximum).
//
// Every kernel reads the sequence length and block table on the device and
// never needs host-side knowledge of tensor contents, so launches are
// graph-capturable and replay correctly with new lengths, pages and KV.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <utility>

#include "pd_device.h"
#include "pd_internal.h"

namespace {

using namespace pdk;

template <int D, int GP>
struct MatchedShared {
  float wmax[2][4][16];  // per-tile maxima, double-buffered by tile parity
  float lsum[4][16];
  int last;
};

// kMode selects the protocol of the partition:
//   kMatched  normalized FP32 partial + LSE, bf16(p) in PV, exp2 with
//             SCALE_LOG2 (matched_splitkv.py:52-98); kFused = true adds the
//             in-kernel merge (below).
//   kBase     the whole context as one partition, FP32 p, natural exp of the
//             scaled scores, output acc / denom in bf16 (kernels.py:10-41).
//   kSplit    the same arithmetic over fixed partitions, storing (m, l, acc)
//             in the reference's units (kernels.py:44-80): m of the scaled
//             scores into `maxima`, l into `lse_out`, unnormalized acc into
//             `partials`.  One workgroup walks every partition of its
//             (kv head, sequence) (grid.x = 1).
//   kSplitPart  kSplit with one workgroup per partition (grid.x = splits), as
//             the reference launches _split (runtime.py:111-113).  Each
//             partition's arithmetic is the walk's, so both write the same
//             bits.
//   kMatchedWalk  kMatched over `wf` consecutive splits of one (kv head,
//             sequence) per workgroup (grid.x = ceil(splits / wf)), for
//             plans with more workgroups than CUs: one resident round of
//             workgroups instead of several.  Each split's arithmetic is
//             kMatched's, so partials and LSEs are the same bits.
// FP32 p goes through the bf16 MFMA as three bf16 terms hi + mid + lo (each
// the RNE bf16 of the previous remainder), which represent p to 2^-27 of its
// value, finer than p's own float32 rounding; with exact bf16 x bf16 products
// and FP32 accumulation, P V is then the FP32 sum the reference computes, in
// another summation order.
//
// kFused = true: after writing its partial, each workgroup releases it at
// device scope and increments counters[b, kh]; the workgroup that completes
// the count acquires, merges all splits of its GQA group into `out` with the
// same arithmetic as lse_merge_kernel, and resets the counter to 0, so the
// counters are zero again when the kernel ends (graph replays need no reset).
//
// A workgroup serves query heads [qb, qb + Gs) of kv head kh: the whole group
// (hs = 1) when it has at most 16 heads, else 16-head slices of it (grid.y =
// Hkv * hs), so the base and fixed-split protocols also cover G > 16.
constexpr int kMatched = 0, kBase = 1, kSplit = 2, kSplitPart = 3, kMatchedWalk = 4;

// Split counters of the fused launch: four per (sequence, kv head), one per
// column slice of the single-tile kernel (the multi-tile kernels use the
// first), each on a 128-byte line of its own, so that the atomics of
// different slices do not queue on one line.
constexpr int kCounterStride = 32;
constexpr int kCountersPerGroup = 4 * kCounterStride;
static_assert(kCountersPerGroup == PD_FUSED_COUNTERS_PER_GROUP, "C ABI counter layout");

// A partition without tokens, written directly: the values the full epilogue
// derives from the untouched state (acc 0, running maximum -inf, denominator
// 0), without its LDS exchange and barriers.  Matched: partial +0, LSE -inf;
// base: output +0 (kernels.py:40); fixed split: acc +0, m -inf, l 0.  Plans
// sized for a table capacity far above the live lengths have mostly such
// partitions.  Not for the fused protocol, whose workgroups must count
// themselves.
template <int D, int kMode>
__device__ __forceinline__ void write_empty_partition(int tid, int b, int Hq, int qb, int Gs,
                                                      int splits, int p, float* partials,
                                                      float* lse_out, uint16_t* out,
                                                      float* maxima) {
  for (int i = tid; i < Gs * D; i += kThreads) {
    const int64_t row = int64_t(b) * Hq + qb + i / D;
    if constexpr (kMode == kBase)
      out[row * D + i % D] = 0;
    else
      partials[(row * splits + p) * D + i % D] = 0.f;
  }
  if (kMode != kBase && tid < Gs) {
    const int64_t orow = (int64_t(b) * Hq + qb + tid) * splits + p;
    if constexpr (kMode == kSplit) {
      maxima[orow] = -INFINITY;
      lse_out[orow] = 0.f;
    } else {
      lse_out[orow] = -INFINITY;
    }
  }
}

template <int D>
struct TileP {
  static constexpr int kTile = 16384 / D;
  // Bytes per head row of P: 8 bytes of padding put the 16 rows of a
  // ds_write_b64 / ds_read_b64 in different banks (row r starts at bank 2r).
  static constexpr int kPitch = 2 * kTile + 8;
  static constexpr int kCols = D / 4;        // output columns per wavefront
  static constexpr int kNBW = kCols / 16;    // 16-column blocks per wavefront
  static constexpr int kKS = kTile / 32;     // 32-token k-steps of PV
};

// f(integral_constant<int, K>) for K = KS... in order.
template <typename F, int... KS>
__device__ __forceinline__ void for_each_step(F&& f, std::integer_sequence<int, KS...>) {
  (f(std::integral_constant<int, KS>{}), ...);
}

// P V of one tile for wavefront w's output columns [w D/4, (w + 1) D/4),
// accumulated into acc (O[head 4(L/16) + r][w D/4 + 16j + L%16] in lane L,
// element r of acc[j]): k-step ks covers tile rows 32ks .. 32ks + 31; lane L
// supplies k = 8(L/16) + e <-> row 32ks + 8(L/16) + e for both operands (as in
// matched_tile_kernel).  The probabilities are in `ps`, one 16-row LDS tile
// per bf16 term; the V rows in `slot`, wavefront x's kTW rows in a kSlot part
// of their own, pieces permuted by vswz.  With kSkipPadRows, the rows of
// padding query heads (qh >= Gs) are neither written (by the caller) nor read:
// their lanes take zeros, which frees LDS bandwidth for the three bf16 terms
// at D = 256 (paired A/B on the edge-coverage batches at D 256 GQA 8:1: 1.8%
// and 2.2% faster); at D 128 (and at D 64, before P V by rows there) the
// four and eight k-steps' masked reads cost more than they save, and for the
// matched protocol's one term they changed nothing (+0.1 to +0.4%).
template <int D, int kTerms>
inline constexpr bool kSkipPadRows = D == 256 && kTerms == 3;

template <int D, int GP, int kTerms>
__device__ __forceinline__ void pv_tile_cols(floatx4_t (&acc)[TileP<D>::kNBW],
                                             const char (*ps)[16 * TileP<D>::kPitch],
                                             const char* slot, int lane, int w, int Gs) {
  using C = Matched<D, GP>;
  using P = TileP<D>;
  const int qh = lane & 15, qg = lane >> 4;
  // Row u = 8qg + qh/4 of a k-step (lo; hi is u + 4), and its place in the
  // slot: wavefront part u / kTW, row u % kTW (u + 4 stays in the same part).
  const int u = 8 * qg + (qh >> 2);
  const uint32_t vb = lds_address(slot) + (u / C::kTW) * C::kSlot + (u % C::kTW) * C::kPitch;
  // D = 64 with three terms multiplies by rows instead (pv_tile_rows).
  static_assert(!(D == 64 && kTerms == 3), "pv_tile_rows");
  auto pv_step = [&](auto KS) __attribute__((always_inline)) {
    constexpr int ks = decltype(KS)::value;
    bf16x8_t a[kTerms];
    u32x4_t pa[kTerms];
    if constexpr (kSkipPadRows<D, kTerms>) {
      // Reads from inline asm under the lane mask (a plain read would be
      // issued for every lane); lds_settle below makes the results wait.
#pragma unroll
      for (int t = 0; t < kTerms; ++t) pa[t] = u32x4_t{0u, 0u, 0u, 0u};
      if (qh < Gs) {
#pragma unroll
        for (int t = 0; t < kTerms; ++t) {
          const uint32_t pr = lds_address(ps[t]) + qh * P::kPitch + (32 * ks + 8 * qg) * 2;
          asm volatile("ds_read2_b64 %0, %1 offset1:1" : "=v"(pa[t]) : "v"(pr));
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < kTerms; ++t) {
        const char* prow = ps[t] + qh * P::kPitch + (32 * ks + 8 * qg) * 2;
        const u32x2_t a0 = *reinterpret_cast<const u32x2_t*>(prow);
        const u32x2_t a1 = *reinterpret_cast<const u32x2_t*>(prow + 8);
        a[t] = __builtin_bit_cast(bf16x8_t, u32x4_t{a0[0], a0[1], a1[0], a1[1]});
      }
    }
    // The transposed reads are issued from inline asm (lds_read_tr_at): the
    // compiler then adds no vmcnt wait of its own for the LDS copies it
    // cannot tell apart from this slot's (the caller's wait covers them), and
    // lds_settle makes the results wait for the reads.
    constexpr int kOff = (32 * ks / C::kTW) * C::kSlot + (32 * ks % C::kTW) * C::kPitch;
    short4_t lo[P::kNBW], hi[P::kNBW];
#pragma unroll
    for (int j = 0; j < P::kNBW; ++j) {
      const uint32_t vj = vb + v_read_offset<D>(w * P::kCols + 16 * j, lane, u % 16);
      lo[j] = lds_read_tr_at<kOff>(vj);
      hi[j] = lds_read_tr_at<kOff + 4 * C::kPitch>(vj);
    }
    lds_settle(lo, hi);
    if constexpr (kSkipPadRows<D, kTerms>) {
#pragma unroll
      for (int t = 0; t < kTerms; ++t) {
        asm volatile("" : "+v"(pa[t]));
        a[t] = __builtin_bit_cast(bf16x8_t, pa[t]);
      }
    }
#pragma unroll
    for (int j = 0; j < P::kNBW; ++j) {
      const bf16x8_t bv = __builtin_bit_cast(
          bf16x8_t, u32x4_t{__builtin_bit_cast(u32x2_t, lo[j])[0], __builtin_bit_cast(u32x2_t, lo[j])[1],
                            __builtin_bit_cast(u32x2_t, hi[j])[0], __builtin_bit_cast(u32x2_t, hi[j])[1]});
#pragma unroll
      for (int t = 0; t < kTerms; ++t)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[t], bv, acc[j], 0, 0, 0);
    }
  };
  for_each_step(pv_step, std::make_integer_sequence<int, P::kKS>{});
}

// P V by rows (D = 64, three bf16 terms): compute wavefront w multiplies the
// probabilities of its own 64 tile rows, still in registers, by all 64 V
// columns, into acc[j] = O_w[head 4qg + r][16j + qh]; the four wavefronts'
// O_w are summed at the partition's end.  pa[s][t] holds bf16 term t (lo,
// mid, hi) of the lane's probabilities of head qh at rows 16g + 4qg + 0..3 of
// its rows for g = 2s (words 0-1) and 2s + 1 (words 2-3), two per word, where
// the scores left them: the A operand of 32-row k-step s (k = 8qg + e <-> row
// 16(2s) + 4qg + e for e < 4, 16(2s + 1) + 4qg + e - 4 above), and the B
// operand is read transposed in the same k order: rows 4qg .. 4qg + 3 and
// 16 + 4qg .. 16 + 4qg + 3 of the k-step (V pieces swizzled by
// vswz<64, true>).  vo[j] is the lane's byte offset for columns 16j ..
// 16j + 15 within its wavefront's rows (v_rows_offsets).  No P goes through
// LDS: at D = 64 the P tile is 16 x 256 and every wavefront read all of it in
// pv_tile_cols.
template <int GP>
__device__ __forceinline__ void pv_tile_rows(floatx4_t (&acc)[4], const u32x4_t (&pa)[2][3],
                                             const char* slot, int w, const uint32_t (&vo)[4]) {
  using C = Matched<64, GP>;
  static_assert(C::kNG == 4 && C::kTW == 64, "D = 64 geometry");
  const uint32_t vb = lds_address(slot) + w * C::kSlot;
  auto step = [&](auto S) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
    constexpr int kLo = 32 * s * C::kPitch, kHi = kLo + 16 * C::kPitch;
    short4_t lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo[j] = lds_read_tr_at<kLo>(vb + vo[j]);
      hi[j] = lds_read_tr_at<kHi>(vb + vo[j]);
    }
    lds_settle(lo, hi);
    bf16x8_t a[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) a[t] = __builtin_bit_cast(bf16x8_t, pa[s][t]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8_t bv = __builtin_bit_cast(
          bf16x8_t, u32x4_t{__builtin_bit_cast(u32x2_t, lo[j])[0], __builtin_bit_cast(u32x2_t, lo[j])[1],
                            __builtin_bit_cast(u32x2_t, hi[j])[0], __builtin_bit_cast(u32x2_t, hi[j])[1]});
#pragma unroll
      for (int t = 0; t < 3; ++t)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[t], bv, acc[j], 0, 0, 0);
    }
  };
  for_each_step(step, std::make_integer_sequence<int, 2>{});
  // The rescale of the next tile reads acc behind a branch (the compiler's
  // wait states there have been too few before).
  mfma_result_barrier(acc);
}

// The lane's byte offsets for pv_tile_rows: row 4qg + qh / 4 of a k-step's
// first 16 (the transposed read's source row of lane 4c + b of its 16-lane
// group is row c of the group's block), columns 16j + 4(qh % 4) .. + 3.
template <int GP>
__device__ __forceinline__ void v_rows_offsets(uint32_t (&vo)[4], int lane) {
  const int qh = lane & 15, qg = lane >> 4;
  const int row = 4 * qg + (qh >> 2);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    vo[j] = uint32_t(row * Matched<64, GP>::kPitch + v_read_offset<64, true>(16 * j, lane, row));
}

// --------------------------------------- multi-tile partition, loader waves
// The partition of every multi-tile plan, for the three protocols (kMode):
// scores on MFMA, the running maxima and denominators of the FP32 online
// softmax, and the P V product split by output columns as in
// matched_tile_kernel: per tile, every compute wavefront writes its bf16
// probabilities (three bf16 terms for the base and fixed-split protocols) to
// LDS, and compute wavefront w multiplies the whole tile's P by V columns
// [w D/4, (w + 1) D/4) (pv_tile_cols).  The accumulator takes D/16 VGPRs, and
// O needs no cross-wave reduction at the end.  At D = 64 in the base and
// fixed-split protocols (three bf16 terms: a 16 x 256 P tile that every
// wavefront would read whole) each wavefront instead multiplies its own rows'
// P, kept in registers, by all 64 columns (pv_tile_rows), and the four
// wavefronts' O are summed where a partition ends (kRowsPV: the paired A/B on
// the edge-coverage batches at D 64 measured x0.963 for hip_base and x0.967
// for hip_splitk, another fp32 summation order).  At D = 64, kHeads = H = 2 or 4
// serves H adjacent kv heads (base and fixed-split protocols): row R of a
// tile is token R / H of kv head H kh + R % H, a token's H rows one contiguous
// read of 128 H bytes; query head e G + g scores only the rows of its own kv
// head (R % H = e), and the other rows get probability 0.
//
// Eight wavefronts: four compute and four only copy K and V rows into LDS
// (buffer_load ... lds).  The LDS below allows one workgroup per CU, so each
// compute wavefront is alone on its SIMD; a wavefront that issues loads
// stands still while the CU's load path takes them (about 64 bytes per clock,
// 64 KiB per tile), so here the loader wavefronts stand still instead, and the
// compute wavefronts issue no global load after the query.  (Four wavefronts
// that loaded for themselves, K two tiles ahead into registers and V into
// LDS, at two workgroups per CU, took 1.17-1.40x the time at D = 256 on few
// long partitions, 1.02-1.06x on full grids, and 1.02-1.04x at D = 64 and
// 128 on full grids.)
//
// LDS: two K and two V stages of 32 KiB (a tile is 16384 / D rows of 2D
// bytes); tile t uses stage t & 1.  K row r of a stage holds its 16-byte
// piece p at position p ^ kswz(r), so the 16 rows of a compute wavefront's
// ds_read_b128 (one piece each) fall on 16 distinct 16-byte bank groups, and
// each loader copy (1 KiB, every eight consecutive lanes one 128-byte line)
// writes one contiguous KiB.  Compute wavefront w's V rows (tile rows kTW w ..
// kTW w + kTW - 1) are loader w's kSlot part of a V stage, pieces permuted by
// vswz.
//
// Schedule, tile t (last to first), around the compute wavefronts' barriers:
//   B1(t)  after QK(t) and the tile maxima.  V stage (t + 1) & 1 is free (P V
//          of tile t + 1 is done): the loaders issue V(t - 1) into it, then
//          wait for V(t) and K(t - 1) and go on to B2(t).
//   B2(t)  before P V of tile t, which needs V(t); QK(t - 1) follows P V with
//          no barrier between them, so K(t - 1) is in LDS too.  K stage t & 1
//          is free since B1(t): the loaders issue K(t - 2) into it.
// Issuing 16 KiB takes a loader about as long as the probabilities take the
// compute wavefronts, so each barrier interval holds the issue of one
// tensor's copies: V between B1 and B2, K between B2 and the next B1,
// alongside P V and QK.  A first barrier B0 covers K(count - 1), issued with
// V(count - 1) and K(count - 2) before it.  Both halves pass the same
// barriers: B0, B1 and B2 of every tile, the fixed-split protocols' barrier
// after the last partition (ti = 0), the one before the epilogue and the
// fused split count's two.
template <int D, int GP, bool kFused, int kMode, int kHeads = 1>
__global__ void __launch_bounds__(2 * kThreads, 1)
cols_loader_kernel(const int32_t* __restrict__ table, const int32_t* __restrict__ lengths,
                   const uint16_t* __restrict__ q, int tsb, int width, int order, int T, int qsb,
                   int qsh, int G, int hs, int Hq, const uint16_t* __restrict__ k,
                   const uint16_t* __restrict__ v, float* __restrict__ partials,
                   float* __restrict__ lse_out, int* __restrict__ counters,
                   uint16_t* __restrict__ out, float* __restrict__ maxima, int Hkv, int splits,
                   float scale, float c, int wf) {
  static_assert(kMode == kMatched || !kFused, "only the matched protocol has a fused merge");
  // The matched protocol's arithmetic (bf16 p, exp2, normalized partial + LSE).
  constexpr bool kMatchedArith = kMode == kMatched || kMode == kMatchedWalk;
  static_assert(kHeads == 1 || !kMatchedArith, "kv-head groups change the tile of the protocol");
  static_assert(kHeads == 1 || ((kHeads == 2 || kHeads == 4) && D == 64), "kv-head groups at D = 64 only");
  using C = Matched<D, GP>;
  using P = TileP<D>;
  constexpr int TILE = C::kTile;        // tile rows: TILE / kHeads tokens of kHeads kv heads
  constexpr int TTOK = TILE / kHeads;   // tokens per tile
  constexpr int kTerms = kMatchedArith ? 1 : 3;
  // D = 64 with three terms: P V by rows (pv_tile_rows), P kept in registers.
  constexpr bool kRowsPV = D == 64 && kTerms == 3;
  constexpr int kStage = TILE * D * 2;  // bytes of one K or V stage
  constexpr int kCopies = C::kDma;      // 1 KiB copies per loader, tensor and tile
  constexpr int kPieces = D / 8;        // 16-byte pieces per K row
  static_assert(4 * C::kSlot == kStage && 4 * 1024 * kCopies == kStage && C::kNG * C::kCH == 8,
                "tile geometry");
  __shared__ MatchedShared<D, GP> sm;
  __shared__ __attribute__((aligned(16))) char ks[2][kStage];
  __shared__ __attribute__((aligned(16))) char vs[2][kStage];
  __shared__ __attribute__((aligned(16))) char ps[kRowsPV ? 1 : kTerms][kRowsPV ? 16 : 16 * P::kPitch];
  __shared__ __attribute__((aligned(16))) int slens[kMaxOrderedBatch + 4];

  // The fixed-split protocol writes the (m, l, acc) of each T-token partition
  // as its tiles are done.  kSplit walks the whole context of its (kv head,
  // sequence) in one workgroup (grid.x = 1), so a sequence's partitions share
  // one workgroup's start and its K / V pipeline; kSplitPart runs the same
  // code over partition blockIdx.x alone.
  //
  // A completed partition goes to global memory through the loader
  // wavefronts: the compute wavefronts leave its acc in `fb` (query head h at
  // fb[h * kFbPitch + c]), its maxima in `fm` and their denominator shares in
  // sm.lsum, and the loaders read them back and store them with 16-byte
  // stores after issuing their next K copies (kSplit holds them in registers
  // and stores several together, below).  A compute wavefront that stored
  // them itself stood still for about 1-2 us per partition (its stores wait
  // behind the loaders' copies), which every wavefront then waited for at
  // the next barrier.
  // kWalk: several partitions per workgroup, [p, p_end) (all of the
  // sequence's for kSplit, whose launch passes wf = splits).
  constexpr bool kWalk = kMode == kSplit || kMode == kMatchedWalk;
  constexpr bool kFlush = kMode == kSplit || kMode == kSplitPart || kMode == kMatchedWalk;
  constexpr int kFbPitch = D + 4;                 // floats per head row of fb
  constexpr int kFbPasses = GP * D >= 1024 ? GP * D / 1024 : 1;  // 16-byte stores per loader lane
  // kRowsPV: one copy of fb per compute wavefront (its O_w), summed by the readers
  // as (w0 + w1) + (w2 + w3); the base protocol's epilogue uses them too.
  constexpr int kFbCopies = kRowsPV ? 4 : 1;
  __shared__ __attribute__((aligned(16))) float fb[kFlush || kRowsPV ? kFbCopies * GP * kFbPitch : 4];
  __shared__ float fm[16];
  constexpr int kEmptyMode = kMatchedArith ? kMatched : (kFlush ? kSplit : kMode);  // write_empty_partition's
  const int p = kWalk ? int(blockIdx.x) * wf : int(blockIdx.x);
  const int p_end = kWalk ? min(p + wf, splits) : p + 1;  // partitions [p, p_end) of this workgroup
  const int kh = blockIdx.y / hs, slice = blockIdx.y % hs;
  const int kvh = kHeads * kh;                      // (first) kv head of this workgroup
  const int qb = kvh * G + 16 * slice;              // first query head of this workgroup
  const int Gs = min(16, kHeads * G - 16 * slice);  // query heads of this workgroup
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = wv >= 4;
  const int w = wv & 3;  // compute wavefront w, or loader w
  const int qh = lane & 15, qg = lane >> 4;
  const int start = p * T;
  OrderedSequence seq{int(blockIdx.z), 0};
  if (order >= 0) seq = ordered_sequence(lengths, int(gridDim.z), int(blockIdx.z), order, slens);
  const int b = seq.b;
  PageWindow<2> pw;
  if (loader) pw.load(table + int64_t(b) * tsb, width, start >> 8, lane);
  const int length = order >= 0 ? seq.length : lengths[b];
  const int end = min(p_end * T, length);
  const int count = end > start ? (end - start + TTOK - 1) / TTOK : 0;
  const int tpp = T / TTOK;  // tiles per partition of the walk
  const int64_t RS = int64_t(Hkv) * D;

  if (loader) {
    if (!kFused && count == 0) return;
    // Copy i of loader w fills KiB 8w + i of the K stage, pieces in position
    // order (piece p of row r at position p ^ kswz(r)), and of V the rows of
    // compute wavefront w.
    int koff[kCopies], voff[kCopies];
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
      const int pos = 64 * (kCopies * w + i) + lane;
      const int row = pos / kPieces;
      koff[i] = (tile_row_elems<D, kHeads>(row, int(RS)) + 8 * ((pos % kPieces) ^ kswz<D>(row))) * 2;
      voff[i] = v_copy_offset<D, GP, kHeads, kRowsPV>(i, lane, w, int(RS));
    }
    pw.settle();
    auto issue = [&](int ti, bool is_k) __attribute__((always_inline)) {
      const int t0 = start + ti * TTOK;
      const TileBuffers buf = tile_buffers(k, v, pw.page(t0), t0, end, RS, kvh, D);
      char* dst = (is_k ? ks[ti & 1] : vs[ti & 1]) + w * kCopies * 1024;
#pragma unroll
      for (int i = 0; i < kCopies; ++i)
        lds_copy16(is_k ? buf.k : buf.v, dst + 1024 * i, is_k ? koff[i] : voff[i]);
    };
    if (count > 0) {
      issue(count - 1, true);
      issue(count - 1, false);
      if (count >= 2) {
        issue(count - 2, true);
        wait_vmcnt<2 * kCopies>();
      } else {
        wait_vmcnt<kCopies>();
      }
      lds_barrier();  // B0
    }
    // The partition flush: loader w's share of a completed partition, read
    // from LDS (inline asm reads: a compiler-placed wait before a plain LDS
    // read would count the copies in flight) and stored after the next K
    // copies are issued.  In-order completion then lets the next wait for K
    // cover the stores too.
    u32x4_t fx[kFbPasses * kFbCopies];  // pass i, copy c at fx[i * kFbCopies + c]
    u32x4_t fd[kMatchedArith ? kFbPasses : 1];  // denominator shares of the pass's head
    uint32_t fmx = 0, fl[4] = {0, 0, 0, 0};
    auto flush_read = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < kFbPasses; ++i) {
        const int f = (i * 256 + w * 64 + lane) * 4;
        const int h = min(f / D, GP - 1);  // rows past GP are never stored
#pragma unroll
        for (int c = 0; c < kFbCopies; ++c)
          fx[i * kFbCopies + c] =
              lds_read16_at(lds_address(reinterpret_cast<const char*>(fb)) +
                            uint32_t(c * GP * kFbPitch + h * kFbPitch + f % D) * 4);
        if constexpr (kMatchedArith) {
          const int hh = h & 15;
#pragma unroll
          for (int x = 0; x < 4; ++x)
            fd[i][x] = lds_read4_at(lds_address(reinterpret_cast<const char*>(&sm.lsum[x][hh])));
        }
      }
      if (w == 0) {
        const int h = lane & 15;
        fmx = lds_read4_at(lds_address(reinterpret_cast<const char*>(fm)) + h * 4);
#pragma unroll
        for (int x = 0; x < 4; ++x)
          fl[x] = lds_read4_at(lds_address(reinterpret_cast<const char*>(&sm.lsum[x][h])));
      }
      lds_wait(fx);
      if constexpr (kMatchedArith) lds_wait(fd);
      asm volatile("" : "+v"(fmx), "+v"(fl[0]), "+v"(fl[1]), "+v"(fl[2]), "+v"(fl[3]));
      if constexpr (kRowsPV) {
        // The partition's accumulators: the four compute wavefronts' rows.
#pragma unroll
        for (int i = 0; i < kFbPasses; ++i) {
          u32x4_t sum;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const auto x = [&](int c) { return __uint_as_float(fx[i * kFbCopies + c][e]); };
            sum[e] = __float_as_uint((x(0) + x(1)) + (x(2) + x(3)));
          }
          fx[i] = sum;
        }
      }
    };
    auto flush_store = [&](int part) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < kFbPasses; ++i) {
        const int f = (i * 256 + w * 64 + lane) * 4;
        const int h = f / D;
        if (h < Gs) {
          const int64_t orow = (int64_t(b) * Hq + qb + h) * splits + part;
          if constexpr (kMatchedArith) {
            // partial = acc * rcp(denominator), as the epilogue below.
            const float den = (__uint_as_float(fd[i][0]) + __uint_as_float(fd[i][1])) +
                              (__uint_as_float(fd[i][2]) + __uint_as_float(fd[i][3]));
            const float inv = rcp_fast(den > 0.f ? den : 1.f);
            fx[i] = u32x4_t{__float_as_uint(__uint_as_float(fx[i][0]) * inv),
                            __float_as_uint(__uint_as_float(fx[i][1]) * inv),
                            __float_as_uint(__uint_as_float(fx[i][2]) * inv),
                            __float_as_uint(__uint_as_float(fx[i][3]) * inv)};
          }
          *reinterpret_cast<u32x4_t*>(partials + orow * D + f % D) = fx[i];
        }
      }
      if (w == 0 && lane < Gs) {
        const int64_t orow = (int64_t(b) * Hq + qb + lane) * splits + part;
        const float den = (__uint_as_float(fl[0]) + __uint_as_float(fl[1])) +
                          (__uint_as_float(fl[2]) + __uint_as_float(fl[3]));
        if constexpr (kMatchedArith) {
          const float safe = den > 0.f ? den : 1.f;
          lse_out[orow] = den > 0.f ? fmaf(__uint_as_float(fmx), scale, ln_fast(safe)) : -INFINITY;
        } else {
          maxima[orow] = __uint_as_float(fmx);
          lse_out[orow] = den;
        }
      }
    };
    // kSplit holds up to kHold completed partitions in the loaders' registers
    // and stores them together, when the hold is full and after the walk's last
    // tile: stored one at a time in the middle of the K / V stream, each
    // partition cost about 2.5 us of the walk at D = 256.  The partitions of a
    // hold are consecutive, hfirst, hfirst - 1, ... (the walk runs backwards).
    constexpr int kHold = kMode != kSplit ? 1 : kFbPasses == 1 ? 16 : kFbPasses == 2 ? 8 : 4;
    u32x4_t hx[kHold][kFbPasses];
    float hm[kHold], hl[kHold];
    int held = 0, hfirst = 0;
    auto store_held = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < kHold; ++j) {
        if (j < held) {
#pragma unroll
          for (int i = 0; i < kFbPasses; ++i) {
            const int f = (i * 256 + w * 64 + lane) * 4;
            const int h = f / D;
            if (h < Gs) {
              const int64_t orow = (int64_t(b) * Hq + qb + h) * splits + hfirst - j;
              *reinterpret_cast<u32x4_t*>(partials + orow * D + f % D) = hx[j][i];
            }
          }
          if (w == 0 && lane < Gs) {
            const int64_t orow = (int64_t(b) * Hq + qb + lane) * splits + hfirst - j;
            maxima[orow] = hm[j];
            lse_out[orow] = hl[j];
          }
        }
      }
      held = 0;
    };
    auto hold = [&](int part) __attribute__((always_inline)) {
      if (held == kHold) store_held();
      if (held == 0) hfirst = part;
      const float den = (__uint_as_float(fl[0]) + __uint_as_float(fl[1])) +
                        (__uint_as_float(fl[2]) + __uint_as_float(fl[3]));
#pragma unroll
      for (int j = 0; j < kHold; ++j) {
        if (j == held) {
#pragma unroll
          for (int i = 0; i < kFbPasses; ++i) hx[j][i] = fx[i];
          hm[j] = __uint_as_float(fmx);
          hl[j] = den;
        }
      }
      ++held;
    };
    auto complete = [&](int part) __attribute__((always_inline)) {
      if constexpr (kMode == kSplit) {
        hold(part);
      } else {
        flush_store(part);
      }
    };
    for (int ti = count - 1; ti >= 0; --ti) {
      lds_barrier();  // B1(ti)
      // The partition that ended with tile ti + 1 is in LDS since B1(ti).
      const bool flushed = kFlush && ti + 1 < count && (ti + 1) % tpp == 0;
      if (ti >= 1) issue(ti - 1, false);
      if (flushed) flush_read();
      if (ti >= 1) {
        wait_vmcnt<kCopies>();
      } else {
        wait_vmcnt<0>();
      }
      lds_barrier();  // B2(ti)
      if (ti >= 2) issue(ti - 2, true);
      if (flushed) complete(p + (ti + 1) / tpp);
      if (kFlush && ti == 0) {
        lds_barrier();  // the last partition's flush
        flush_read();
        complete(p);
        if constexpr (kMode == kSplit) store_held();
      }
    }
    if constexpr (!kFlush) lds_barrier();  // epilogue
    if constexpr (kFused) {
      __syncthreads();  // the split count's two barriers
      __syncthreads();
    }
    return;
  }

  if (!kFused && count == 0) {
    for (int pp = p; pp < p_end; ++pp)
      write_empty_partition<D, kEmptyMode>(tid, b, Hq, qb, Gs, splits, pp, partials, lse_out,
                                           out, maxima);
    // The walk's merged output of an empty sequence is 0 (no live partition),
    // and so is the directly written output of a one-split matched plan.
    if ((kMode == kSplit || kMode == kMatched) && out != nullptr)
      write_empty_partition<D, kBase>(tid, b, Hq, qb, Gs, splits, 0, partials, lse_out, out,
                                      maxima);
    return;
  }
  bf16x8_t qf[C::kCH];
  {
    const bool live = qh < Gs;
    const uint16_t* qrow = q + int64_t(b) * qsb + int64_t(qb + (live ? qh : 0)) * qsh + 8 * qg;
#pragma unroll
    for (int ch = 0; ch < C::kCH; ++ch)
      qf[ch] = __builtin_bit_cast(bf16x8_t, live ? load16(qrow + 32 * ch) : u32x4_t{0, 0, 0, 0});
  }
  // Lane (qh, qg) reads piece qg + 4ch of K row kTW w + 16g + qh for 16-row
  // group g and k-chunk ch; a tile's reads are issued once its rows are in
  // LDS (after P V of the tile before it) and waited for before its QK
  // products.
  uint32_t kaddr[C::kNG * C::kCH];
#pragma unroll
  for (int g = 0; g < C::kNG; ++g) {
    const int row = w * C::kTW + 16 * g + qh;
#pragma unroll
    for (int ch = 0; ch < C::kCH; ++ch)
      kaddr[g * C::kCH + ch] =
          lds_address(ks[0]) + row * (2 * D) + (((qg + 4 * ch) ^ kswz<D>(row)) * 16);
  }
  u32x4_t kr[C::kNG * C::kCH];
  auto read_k = [&](int ti) __attribute__((always_inline)) {
    const uint32_t stage = (ti & 1) * kStage;
#pragma unroll
    for (int i = 0; i < C::kNG * C::kCH; ++i) kr[i] = lds_read16_at(kaddr[i] + stage);
  };

  // O[head 4*qg + r][64w + 16j + qh] over the tile's rows; with kRowsPV,
  // O_w[head 4*qg + r][16j + qh] over this wavefront's rows only.
  constexpr int kAccB = kRowsPV ? 4 : P::kNBW;
  floatx4_t acc[kAccB];
#pragma unroll
  for (int j = 0; j < kAccB; ++j) acc[j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  u32x4_t pa[kRowsPV ? C::kNG / 2 : 1][3];  // kRowsPV: the tile's P terms (pv_tile_rows)
  uint32_t vo[4] = {0u, 0u, 0u, 0u};
  if constexpr (kRowsPV) v_rows_offsets<GP>(vo, lane);
  // kRowsPV: O of head h, column col, as (O_0 + O_1) + (O_2 + O_3) from the
  // wavefronts' copies in fb (the loaders' flush_read sums the same way).
  auto rows_sum = [&](int h, int col) __attribute__((always_inline)) {
    const float* x = fb + h * kFbPitch + col;
    constexpr int kCopy = GP * kFbPitch;
    return (x[0] + x[kCopy]) + (x[2 * kCopy] + x[3 * kCopy]);
  };
  float m4[4];             // running max of heads 4*qg + r
#pragma unroll
  for (int r = 0; r < 4; ++r) m4[r] = -INFINITY;
  float m_own = -INFINITY;  // running max of head qh
  // The lane's kv head in a group of kHeads (e), as bit masks for the score
  // select, and the scale in a register of its own (a kernel argument the
  // compiler would otherwise fetch again in every tile).
  const int e = kHeads > 1 ? min(qh / G, kHeads - 1) : 0;
  uint32_t emask[kHeads > 1 ? kHeads : 1];
#pragma unroll
  for (int r = 0; r < (kHeads > 1 ? kHeads : 1); ++r) emask[r] = r == e ? 0xffffffffu : 0u;
  float scale_v = scale;
  asm volatile("" : "+v"(scale_v));
  float l_own = 0.f;        // this lane's share of head qh's denominator
  // The walk with an output (out != nullptr) also merges the partitions as it
  // completes them, with ml_online_merge_kernel's arithmetic (ml_step): running
  // maxima mM of heads 4 qg + r, merged accumulators mO (the lane's columns of
  // acc) and totals mT.  A partition's denominator needs every wavefront's
  // share (sm.lsum), so its steps mS wait (`pending`) for the next barrier
  // every wavefront passes: B1 of the next tile, or the last partition's own.
  // The next flush writes sm.lsum after B2 of the following tile, when these
  // reads (before the wavefront reaches B2) are done.
  const bool merge_out = kMode == kSplit && out != nullptr;
  bool pending = false;
  floatx4_t mO[P::kNBW];
  float mM[4], mT[4];
  MlStep mS[4];
  if (kMode == kSplit) {
#pragma unroll
    for (int j = 0; j < P::kNBW; ++j) mO[j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      mM[r] = -INFINITY;
      mT[r] = 0.f;
      mS[r] = MlStep{1.f, 0.f, false};
    }
  }
  auto merge_denominators = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * qg + r;
      const float den = (sm.lsum[0][h] + sm.lsum[1][h]) + (sm.lsum[2][h] + sm.lsum[3][h]);
      if (mS[r].live) mT[r] = fmaf(den, mS[r].b, mT[r] * mS[r].a);
      // kRowsPV: the partition's accumulators are in fb only after this barrier too.
      if constexpr (kRowsPV) {
        if (mS[r].live && h < Gs)
          mO[0][r] = fmaf(rows_sum(h, w * P::kCols + qh), mS[r].b, mO[0][r] * mS[r].a);
      }
    }
  };

  if (count > 0) {
    lds_barrier();  // B0
    read_k(count - 1);
  }
  for (int ti = count - 1; ti >= 0; --ti) {
    // ---- scores and the tile maxima
    const int nvalid = end - (start + ti * TTOK);
    lds_wait(kr);
    floatx4_t s[C::kNG];
#pragma unroll
    for (int g = 0; g < C::kNG; ++g) {
      s[g] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ch = 0; ch < C::kCH; ++ch)
        s[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, kr[g * C::kCH + ch]), qf[ch], s[g], 0, 0, 0);
    }
    mfma_result_barrier(s);
    // kv-head groups: row R = 16 g + 4 qg + r of a wavefront's rows holds kv
    // head R % H, so query head qh (kv head e) scores live rows only at
    // r = e + H i, i < kLive; every other score of the lane would be -inf
    // (probability exactly 0) and is not formed.  x[g][i] is the lane's live
    // score at r = e + H i (-inf past the end), in the reference's units;
    // padding query lanes (qh >= H G) take the last head's rows.
    constexpr int kLive = kHeads > 1 ? 4 / kHeads : 1;
    float x[kHeads > 1 ? C::kNG : 1][kLive];
    if constexpr (kHeads > 1) {
#pragma unroll
      for (int g = 0; g < C::kNG; ++g) {
#pragma unroll
        for (int i = 0; i < kLive; ++i) {
          // s[g][e + H i] by bit masks (a select on the lane's e became branches)
          uint32_t vb = 0;
#pragma unroll
          for (int r = i * kHeads; r < i * kHeads + kHeads; ++r)
            vb |= __float_as_uint(s[g][r]) & emask[r - i * kHeads];
          float v = __uint_as_float(vb);
          // Scores in the reference's units: dot(q, k) * SCALE (kernels.py:30).
          v *= scale_v;
          const int tok = (w * C::kTW + 16 * g + 4 * qg + e + kHeads * i) / kHeads;
          x[g][i] = tok >= nvalid ? -INFINITY : v;
        }
      }
    } else {
      if constexpr (!kMatchedArith) {
        // Scores in the reference's units: dot(q, k) * SCALE (kernels.py:30).
#pragma unroll
        for (int g = 0; g < C::kNG; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[g][r] *= scale_v;
      }
      if (nvalid < TILE) {
#pragma unroll
        for (int g = 0; g < C::kNG; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (w * C::kTW + 16 * g + 4 * qg + r >= nvalid) s[g][r] = -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int g = 0; g < C::kNG; ++g) {
      if constexpr (kHeads > 1) {
#pragma unroll
        for (int i = 0; i < kLive; ++i) mx = fmaxf(mx, x[g][i]);
      } else {
        mx = fmaxf(fmaxf(mx, fmaxf(s[g][0], s[g][1])), fmaxf(s[g][2], s[g][3]));
      }
    }
    mx = max_rows(mx);
    float (*wm)[16] = sm.wmax[ti & 1];
    if (lane < 16) wm[w][lane] = mx;
    lds_barrier();  // B1(ti)
    if constexpr (kMode == kSplit) {
      // The denominators of the partition flushed after the previous tile
      // were written to LDS before this barrier.
      if (pending) {
        merge_denominators();
        pending = false;
      }
    }

    // ---- probabilities, P to LDS (lo, mid, hi for the FP32 probabilities of
    // the base / split protocols), rescale of O
    float alpha[4];
    bool moved = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * qg + r;
      const float tm = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
      const float mn = fmaxf(m4[r], tm);
      moved |= mn != m4[r];
      alpha[r] = kMatchedArith ? exp2_fast((m4[r] - mn) * c) : exp_fast(m4[r] - mn);
      m4[r] = mn;
    }
    const float tm = fmaxf(fmaxf(wm[0][qh], wm[1][qh]), fmaxf(wm[2][qh], wm[3][qh]));
    const float mn = fmaxf(m_own, tm);
    const float a_own = kMatchedArith ? exp2_fast((m_own - mn) * c) : exp_fast(m_own - mn);
    m_own = mn;
    const float neg_mc = -(mn * c);
    float psum = 0.f;
#pragma unroll
    for (int g = 0; g < C::kNG; ++g) {
      if constexpr (kHeads > 1) {
        // The live probabilities in row order, as three bf16 terms each, at
        // positions r = e + H i of the lane's four rows (zero elsewhere).
        const int pofs = qh * P::kPitch + (w * C::kTW + 16 * g + 4 * qg) * 2;
        uint32_t t3[3][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}};
#pragma unroll
        for (int i = 0; i < kLive; ++i) {
          const float pr = exp_fast(x[g][i] - mn);
          psum += pr;
          const uint32_t hi = pack_bf16(pr, 0.f);
          const float r0 = pr - bf16_lo(hi);
          const uint32_t mid = pack_bf16(r0, 0.f);
          const uint32_t lo = pack_bf16(r0 - bf16_lo(mid), 0.f);
          const uint32_t terms[3] = {lo, mid, hi};
          const int pos = e + kHeads * i;  // 0..3
#pragma unroll
          for (int t = 0; t < 3; ++t) {
            const uint32_t word = (pos & 1) ? terms[t] << 16 : terms[t];
            if constexpr (kHeads == 4) {
              t3[t][0] = pos < 2 ? word : 0u;
              t3[t][1] = pos < 2 ? 0u : word;
            } else {
              t3[t][i] = word;
            }
          }
        }
        if constexpr (kRowsPV) {
#pragma unroll
          for (int t = 0; t < 3; ++t) {
            pa[g >> 1][t][2 * (g & 1)] = qh < Gs ? t3[t][0] : 0u;
            pa[g >> 1][t][2 * (g & 1) + 1] = qh < Gs ? t3[t][1] : 0u;
          }
        } else {
#pragma unroll
          for (int t = 0; t < 3; ++t)
            *reinterpret_cast<u32x2_t*>(ps[t] + pofs) =
                u32x2_t{qh < Gs ? t3[t][0] : 0u, qh < Gs ? t3[t][1] : 0u};
        }
        continue;
      }
      float pr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = kMatchedArith ? exp2_fast(fmaf(s[g][r], c, neg_mc)) : exp_fast(s[g][r] - mn);
        psum += pr[r];
      }
      // P[head qh][tile rows kTW w + 16g + 4qg .. +3] into row qh of each
      // term's LDS tile.
      const int pofs = qh * P::kPitch + (w * C::kTW + 16 * g + 4 * qg) * 2;
      if constexpr (kMatchedArith) {
        *reinterpret_cast<u32x2_t*>(ps[0] + pofs) =
            u32x2_t{qh < Gs ? pack_bf16(pr[0], pr[1]) : 0u, qh < Gs ? pack_bf16(pr[2], pr[3]) : 0u};
      } else {
        uint32_t t3[3][2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const uint32_t hi = pack_bf16(pr[2 * h2], pr[2 * h2 + 1]);
          const float r0 = pr[2 * h2] - bf16_lo(hi), r1 = pr[2 * h2 + 1] - bf16_hi(hi);
          const uint32_t mid = pack_bf16(r0, r1);
          const uint32_t lo = pack_bf16(r0 - bf16_lo(mid), r1 - bf16_hi(mid));
          t3[0][h2] = qh < Gs ? lo : 0u;
          t3[1][h2] = qh < Gs ? mid : 0u;
          t3[2][h2] = qh < Gs ? hi : 0u;
        }
        if constexpr (kRowsPV) {
#pragma unroll
          for (int t = 0; t < 3; ++t) {
            pa[g >> 1][t][2 * (g & 1)] = t3[t][0];
            pa[g >> 1][t][2 * (g & 1) + 1] = t3[t][1];
          }
        } else if (!kSkipPadRows<D, kTerms> || qh < Gs) {
#pragma unroll
          for (int t = 0; t < 3; ++t)
            *reinterpret_cast<u32x2_t*>(ps[t] + pofs) = u32x2_t{t3[t][0], t3[t][1]};
        }
      }
    }
    l_own = l_own * a_own + psum;
    if (ti != count - 1 && __builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
      for (int j = 0; j < kAccB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] *= alpha[r];
    }
    lds_barrier();  // B2(ti): P rows written, V(ti) and K(ti - 1) in LDS
    if constexpr (kRowsPV)
      pv_tile_rows<GP>(acc, pa, vs[ti & 1], w, vo);
    else
      pv_tile_cols<D, GP, kTerms>(acc, ps, vs[ti & 1], lane, w, Gs);
    if (ti > 0) read_k(ti - 1);

    if constexpr (kFlush) {
      // After tile ti, the first tile of partition p + ti / tpp, that
      // partition is complete: its (m, l, acc) go to LDS for the loaders to
      // store (kernels.py:77-80), l as per-wavefront shares, and the running
      // state restarts for the partition before it.  The copies of the next
      // tiles stay in flight, and only the last partition takes a barrier of
      // its own.
      if (ti % tpp == 0) {
        const float l = sum_rows(l_own);
        if (lane < 16) sm.lsum[w][lane] = l;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int h = 4 * qg + r;
          if (h >= Gs) break;
          // kRowsPV: this wavefront's O_w, all columns, into its copy of fb.
          float* row = fb + (kRowsPV ? w * GP * kFbPitch : w * P::kCols) + h * kFbPitch + qh;
#pragma unroll
          for (int j = 0; j < kAccB; ++j) row[16 * j] = acc[j][r];
          if (w == 0 && qh == 0) fm[h] = m4[r];
        }
        if (merge_out) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            mS[r] = ml_step(m4[r], mM[r]);
            // kRowsPV: merged after the next barrier (merge_denominators).
            if (!kRowsPV && mS[r].live) {
#pragma unroll
              for (int j = 0; j < P::kNBW; ++j) mO[j][r] = fmaf(acc[j][r], mS[r].b, mO[j][r] * mS[r].a);
            }
          }
        }
        // The loaders store the partition after the next tile's B1 barrier,
        // or after one more barrier for the last partition; the merged
        // totals take its denominators then too.
        pending = merge_out;
        if (ti == 0) {
          lds_barrier();
          if (merge_out) merge_denominators();
        }
#pragma unroll
        for (int j = 0; j < kAccB; ++j) acc[j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < 4; ++r) m4[r] = -INFINITY;
        m_own = -INFINITY;
        l_own = 0.f;
      }
    }
  }
  // No K read is in flight here (tile 0 issues none), but the compiler does
  // not know that the inline-asm reads are asynchronous: its control-flow graph
  // has an exit edge right after read_k, where it would reuse their registers
  // with no wait.  This wait (free: nothing is outstanding) makes every path
  // to such a reuse pass a wait for the reads.
  lds_wait(kr);

  if constexpr (kWalk) {
    // Partitions past the sequence's last token are empty.
    for (int pp = (end + T - 1) / T; pp < p_end; ++pp)
      write_empty_partition<D, kEmptyMode>(tid, b, Hq, qb, Gs, splits, pp, partials, lse_out,
                                           out, maxima);
    if (merge_out) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = 4 * qg + r;
        if (h >= Gs) break;
        const float inv = 1.f / (mT[r] > 0.f ? mT[r] : 1.f);
        uint16_t* dst = out + (int64_t(b) * Hq + qb + h) * D + w * P::kCols + qh;
#pragma unroll
        for (int j = 0; j < P::kNBW; ++j) dst[16 * j] = uint16_t(bf16_bits(mO[j][r] * inv));
      }
    }
    return;
  }
  if constexpr (kFlush) return;  // partition p was written by the flush after its first tile

  // ---- epilogue: denominators over the waves; O needs no reduction (with
  // kRowsPV, the sum of the wavefronts' copies in fb)
  const float l = sum_rows(l_own);
  if (lane < 16) sm.lsum[w][lane] = l;
  if constexpr (kRowsPV) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * qg + r;
      if (h >= Gs) break;
      float* row = fb + w * GP * kFbPitch + h * kFbPitch + qh;
#pragma unroll
      for (int j = 0; j < kAccB; ++j) row[16 * j] = acc[j][r];
    }
  }
  lds_barrier();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * qg + r;
    if (h >= Gs) break;
    const float den = (sm.lsum[0][h] + sm.lsum[1][h]) + (sm.lsum[2][h] + sm.lsum[3][h]);
    const float safe = den > 0.f ? den : 1.f;
    const int col = w * P::kCols + qh;
    if constexpr (kMode == kBase) {
      // acc / denom, 0 for an empty sequence (kernels.py:40).
      uint16_t* dst = out + (int64_t(b) * Hq + qb + h) * D + col;
      if constexpr (kRowsPV) {
        static_assert(P::kNBW == 1, "one 16-column block per wavefront at D = 64");
        dst[0] = uint16_t(bf16_bits(rows_sum(h, col) / safe));
      } else {
#pragma unroll
        for (int j = 0; j < P::kNBW; ++j) dst[16 * j] = uint16_t(bf16_bits(acc[j][r] / safe));
      }
    } else {
      const int64_t orow = (int64_t(b) * Hq + qb + h) * splits + p;
      const float inv = rcp_fast(safe);
      const float lv = den > 0.f ? fmaf(m4[r], scale, ln_fast(safe)) : -INFINITY;
      if constexpr (kFused) {
        // Device-scope stores (global_store sc1): written through to the
        // coherence point, so another XCD can read them without any L2 flush.
#pragma unroll
        for (int j = 0; j < P::kNBW; ++j)
          __hip_atomic_store(partials + orow * D + col + 16 * j, acc[j][r] * inv, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        if (w == 0 && qh == 0)
          __hip_atomic_store(lse_out + orow, lv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
#pragma unroll
        for (int j = 0; j < P::kNBW; ++j) partials[orow * D + col + 16 * j] = acc[j][r] * inv;
        if (w == 0 && qh == 0) lse_out[orow] = lv;
        if (out != nullptr) {
          // A plan of one split (out is passed only then): its LSE merge
          // (matched_splitkv.py:101-127) weighs the split by
          // exp(lse - (ln(exp(lse - lse)) + lse)) = exp2(0) = 1 exactly, so
          // it writes bf16(fma(1, partial, +0)), which is bf16(partial + 0)
          // (-0 becomes +0); an empty split (lse -inf) weighs 0 and gives 0.
          uint16_t* dst = out + (int64_t(b) * Hq + qb + h) * D + col;
#pragma unroll
          for (int j = 0; j < P::kNBW; ++j)
            dst[16 * j] = uint16_t(bf16_bits(den > 0.f ? acc[j][r] * inv + 0.f : 0.f));
        }
      }
    }
  }

  if constexpr (kFused) {
    // Split-completion count.  Every partial and LSE value exchanged between
    // workgroups is written and read with device-scope (sc1) accesses.  Each
    // compute wavefront waits until its own stores have completed (vmcnt(0):
    // written through to the coherence point), then the barrier orders the
    // four wavefronts' completed stores before thread 0 increments the
    // counter; the loader wavefronts pass the two barriers and leave.  The
    // last workgroup issues its loads only after its increment returned
    // splits - 1, i.e. after every other workgroup's stores completed, and
    // those loads are device-scope, so they are served from the coherence
    // point rather than from a line this XCD's caches may hold from an
    // earlier call.  No cache-wide writeback or invalidate is needed, so the
    // KV tiles other calls keep in L2 stay resident.  Compute wavefront w
    // merges query heads w, w + 4, ... of the group; each lane owns D / 64
    // consecutive columns, as in lse_merge_kernel's wavefronts.
    int* counter = counters + (int64_t(b) * Hkv + kh) * kCountersPerGroup;  // the first slot
    wait_memory();
    __syncthreads();
    if (tid == 0)
      sm.last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                splits - 1;
    __syncthreads();
    if (!sm.last) return;
    const int64_t row0 = int64_t(b) * Hq + kh * G;
    constexpr int kV = D / 64;
    for (int hh = __builtin_amdgcn_readfirstlane(w); hh < G; hh += 4) {
      float w0 = 0.f, w1 = 0.f, mrg[kV];
      merge_splits<kV, kCoherentAux>(
          partials + (row0 + hh) * splits * D, D, lane * kV, splits,
          [&] {
            lse_weights<kCoherentAux>(lse_out + (row0 + hh) * splits, splits,
                                      plan_lse_lanes(splits, D), lane, w0, w1);
          },
          [&](int s0, int j) { return wave_weight(w0, w1, s0 + j); }, mrg);
      uint16_t* dst = out + (row0 + hh) * D + lane * kV;
#pragma unroll
      for (int e = 0; e < kV; ++e) dst[e] = uint16_t(bf16_bits(mrg[e]));
    }
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ----------------------------------------------------- single-tile partition
// The same partial + LSE as cols_loader_kernel for plans whose splits
// are exactly one tile (tokens_per_split == 16384 / D: the headline D=256
// plan of 64-token splits, and every plan of small contexts).  With a single
// tile there is no running maximum to carry, so the workgroup splits the PV
// product by output columns instead of by tokens: after the QK scores and the
// tile maximum, every wavefront writes its bf16 probabilities to LDS, and
// wavefront w then multiplies the whole tile's P by V columns
// [w*D/4, (w+1)*D/4) on v_mfma_f32_16x16x32_bf16.  That needs one more barrier
// but no cross-wave reduction of O at the end, and half the PV instructions
// of a 16-token grouping at D=256.  With one tile per workgroup there are no
// later loads to hide, so the four wavefronts load for themselves (no loader
// wavefronts) and two workgroups share a CU.  Scores, maxima, probabilities,
// denominators and LSEs are computed as cols_loader_kernel computes them, and
// P V in the same k-step order.
//
// kFused = true also merges, in the same launch, with the work of the merge
// spread over the column slices the wavefronts already own.  Wavefront w of
// every split writes its columns [w*D/4, (w+1)*D/4) of the partials and the
// group's LSEs with device-scope stores, waits for its own stores to
// complete, and increments counters[(b * Hkv + kh) * 4 + w].  The wavefront
// whose increment returns splits - 1 is the last for its slice: every split's
// slice and LSEs are then complete, and it merges that slice for the whole
// GQA group (merge_group_column, device-scope loads) and resets the counter
// to 0.  So four wavefronts, usually on four CUs, share a group's merge, each
// reading a quarter of its partials, with no workgroup barrier and no cache
// writeback or invalidate.  The output is bit-identical to lse_merge_kernel's.

// Shape of the fused merge of one column slice (D/4 columns of G <= GP heads):
// kNC 4-column chunks per lane, kBatch splits per batch of loads.
template <int D, int GP>
struct FusedMerge {
  static constexpr int kNC = GP * D / 1024 > 1 ? GP * D / 1024 : 1;
  // 20 rather than 24 at kNC = 2 (D 256 with 5-8 query heads): 24 spilled
  // 20 bytes per lane to scratch there, 20 needs 229 VGPRs and none.
  static constexpr int kBatch = kNC == 2 ? 20 : 48 / kNC;
};

template <int D, int GP, bool kFused>
__global__ void __launch_bounds__(kThreads, 2)
matched_tile_kernel(const int32_t* __restrict__ table, const int32_t* __restrict__ lengths,
                    const uint16_t* __restrict__ q, int tsb, int width, int qsb, int qsh, int G,
                    int Hq, int splits, const uint16_t* __restrict__ k,
                    const uint16_t* __restrict__ v, float* __restrict__ partials,
                    float* __restrict__ lse_out, int Hkv, float scale, float c,
                    int* __restrict__ counters, uint16_t* __restrict__ out) {
  using C = Matched<D, GP>;
  using P = TileP<D>;
  constexpr int TILE = C::kTile;
  // The slices are published with device-scope (sc1) stores and read back with
  // device-scope loads: the merging wavefront may run on another XCD, whose L2
  // is not coherent with this one's.
  constexpr int kScope = __HIP_MEMORY_SCOPE_AGENT;
  __shared__ float wmax[4][16];
  __shared__ float lsum[4][16];
  __shared__ __attribute__((aligned(16))) char vs[4 * C::kSlot];
  __shared__ __attribute__((aligned(16))) char ps[16 * P::kPitch];
  // Fused merge: each wavefront's merge weights, [GP][128] floats.
  __shared__ __attribute__((aligned(16))) float wsm[kFused ? 4 * 128 * GP : 4];

  const int p = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qh = lane & 15, qg = lane >> 4;
  const int start = p * TILE;
  PageWindow<1> pw;  // entry 0 of lane 0 is the tile's page
  pw.load(table + int64_t(b) * tsb, width, start >> 8, lane);
  const int length = lengths[b];
  const int end = min(start + TILE, length);
  const int64_t RS = int64_t(Hkv) * D;
  const int64_t row0 = (int64_t(b) * Hq + kh * G) * splits + p;  // (head 0 of the group, p)
  // Wait for the table entry here, before the branch on the length: otherwise
  // the compiler sinks the table load below the branch and the first KV loads
  // wait for two memory round trips (length, then table) instead of one.
  pw.settle();

  // Fused protocol, after this wavefront's slice and LSEs were stored with
  // device-scope stores: count the slice, and merge it if it was the last.
  auto count_and_merge = [&]() {
    wait_memory();
    int* counter = counters + (int64_t(b) * Hkv + kh) * kCountersPerGroup + w * kCounterStride;
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, kScope);
    old = __builtin_amdgcn_readlane(old, 0);
    if (old != splits - 1) return;
    const int64_t grow = int64_t(b) * Hq + kh * G;  // first query head of the group
    using M = FusedMerge<D, GP>;
    merge_group_chunks<GP, M::kNC, M::kBatch, kCoherentAux>(
        partials + grow * splits * D, lse_out + grow * splits, out + grow * D, G, splits, D,
        plan_lse_lanes(splits, D), w * P::kCols, P::kCols, wsm + w * 128 * GP, lane);
    if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, kScope);
  };

  if (end <= start) {
    // Empty split: partial 0 (acc 0 times rcp(1)) and LSE -inf, as the
    // general kernel writes for count == 0.
    if constexpr (kFused) {
      // Each wavefront publishes its own column slice and LSEs.
      if (lane < P::kCols)
        for (int h = 0; h < G; ++h)
          __hip_atomic_store(partials + (row0 + int64_t(h) * splits) * D + w * P::kCols + lane,
                             0.f, __ATOMIC_RELAXED, kScope);
      if (lane < G)
        __hip_atomic_store(lse_out + row0 + int64_t(lane) * splits, -INFINITY, __ATOMIC_RELAXED,
                           kScope);
      count_and_merge();
    } else {
      for (int i = tid; i < G * D; i += kThreads)
        partials[(row0 + int64_t(i / D) * splits) * D + i % D] = 0.f;
      if (tid < G) lse_out[row0 + int64_t(tid) * splits] = -INFINITY;
    }
    return;
  }

  bf16x8_t qf[C::kCH];
  {
    const bool live = qh < G;
    const uint16_t* qrow =
        q + int64_t(b) * qsb + int64_t(kh * G + (live ? qh : 0)) * qsh + 8 * qg;
#pragma unroll
    for (int ch = 0; ch < C::kCH; ++ch)
      qf[ch] = __builtin_bit_cast(bf16x8_t, live ? load16(qrow + 32 * ch) : u32x4_t{0, 0, 0, 0});
  }
  const int kl = kline_offset(lane, int(RS)) + w * C::kTW * int(RS) * 2;
  int voff[C::kDma];
#pragma unroll
  for (int i = 0; i < C::kDma; ++i) voff[i] = v_copy_offset<D, GP>(i, lane, w, int(RS));

  KTile<D, GP> R;
  {
    const TileBuffers buf = tile_buffers(k, v, pw.page(start), start, end, RS, kh, D);
    ktile_load(R, buf.k, kl, int(RS));
#pragma unroll
    for (int i = 0; i < C::kDma; ++i) lds_copy16(buf.v, vs + w * C::kSlot + 1024 * i, voff[i]);
  }
  // Every K and V load of the tile is issued before the K rearrangement, which
  // waits for K.
  __builtin_amdgcn_sched_barrier(0);
  ktile_to_mfma(R, lane);

  // ---- scores of this wavefront's tokens, tile maximum per head
  const int nvalid = end - start;
  floatx4_t s[C::kNG];
#pragma unroll
  for (int g = 0; g < C::kNG; ++g) {
    s[g] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ch = 0; ch < C::kCH; ++ch)
      s[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, R.k[g][ch]),
                                                      qf[ch], s[g], 0, 0, 0);
  }
  mfma_result_barrier(s);
  if (nvalid < TILE) {
#pragma unroll
    for (int g = 0; g < C::kNG; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (w * C::kTW + 16 * g + 4 * qg + r >= nvalid) s[g][r] = -INFINITY;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int g = 0; g < C::kNG; ++g)
    mx = fmaxf(fmaxf(mx, fmaxf(s[g][0], s[g][1])), fmaxf(s[g][2], s[g][3]));
  mx = max_rows(mx);
  if (lane < 16) wmax[w][lane] = mx;
  lds_barrier();
  // m' = max(-inf, tile max) = the tile maximum (matched_splitkv.py:77-78).
  const float m_own = fmaxf(fmaxf(wmax[0][qh], wmax[1][qh]), fmaxf(wmax[2][qh], wmax[3][qh]));
  const float neg_mc = -(m_own * c);
  float psum = 0.f;
#pragma unroll
  for (int g = 0; g < C::kNG; ++g) {
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = exp2_fast(fmaf(s[g][r], c, neg_mc));
      psum += pr[r];
    }
    // P[head qh][tokens w*kTW + 16g + 4qg .. +3] into the head's LDS row.
    const u32x2_t pb{qh < G ? pack_bf16(pr[0], pr[1]) : 0u, qh < G ? pack_bf16(pr[2], pr[3]) : 0u};
    *reinterpret_cast<u32x2_t*>(ps + qh * P::kPitch + (w * C::kTW + 16 * g + 4 * qg) * 2) = pb;
  }
  const float l = sum_rows(psum);
  if (lane < 16) lsum[w][lane] = l;
  __syncthreads();  // P rows, denominators and every wavefront's V rows are in LDS

  // ---- PV: O[heads][this wavefront's columns] over the whole tile.  k-step
  // ks covers tokens 32ks .. 32ks+31; lane L supplies k = 8(L/16) + e <->
  // token 32ks + 8(L/16) + e for both operands.
  floatx4_t acc[P::kNBW];
#pragma unroll
  for (int j = 0; j < P::kNBW; ++j) acc[j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < P::kKS; ++ks) {
    // Two 8-byte reads: the 8-byte row padding keeps them bank-conflict free
    // but leaves odd rows off 16-byte alignment.
    const char* prow = ps + qh * P::kPitch + (32 * ks + 8 * qg) * 2;
    const u32x2_t a0 = *reinterpret_cast<const u32x2_t*>(prow);
    const u32x2_t a1 = *reinterpret_cast<const u32x2_t*>(prow + 8);
    const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4_t{a0[0], a0[1], a1[0], a1[1]});
    const int t_lo = 32 * ks + 8 * qg + (qh >> 2), t_hi = t_lo + 4;
    const char* lo_row = vs + (t_lo / C::kTW) * C::kSlot + (t_lo % C::kTW) * C::kPitch;
    const char* hi_row = vs + (t_hi / C::kTW) * C::kSlot + (t_hi % C::kTW) * C::kPitch;
#pragma unroll
    for (int j = 0; j < P::kNBW; ++j) {
      const int cb = v_read_offset<D>(w * P::kCols + 16 * j, lane, 8 * (qg & 1) + (qh >> 2));
      const short4_t lo = lds_read_tr(lo_row + cb);
      const short4_t hi = lds_read_tr(hi_row + cb);
      const bf16x8_t bv = __builtin_bit_cast(
          bf16x8_t, u32x4_t{__builtin_bit_cast(u32x2_t, lo)[0], __builtin_bit_cast(u32x2_t, lo)[1],
                            __builtin_bit_cast(u32x2_t, hi)[0], __builtin_bit_cast(u32x2_t, hi)[1]});
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bv, acc[j], 0, 0, 0);
    }
  }

  // ---- epilogue: lane L holds O[head 4*qg + r][w*D/4 + 16j + qh]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * qg + r;
    if (h >= G) break;
    const float den = (lsum[0][h] + lsum[1][h]) + (lsum[2][h] + lsum[3][h]);
    const float safe = den > 0.f ? den : 1.f;
    const float inv = rcp_fast(safe);
    float* dst = partials + (row0 + int64_t(h) * splits) * D + w * P::kCols + qh;
    const bool lse_lane = kFused ? qh == 0 : (w == 0 && qh == 0);
    float lv = 0.f;
    if (lse_lane) {
      const float mh = fmaxf(fmaxf(wmax[0][h], wmax[1][h]), fmaxf(wmax[2][h], wmax[3][h]));
      lv = den > 0.f ? fmaf(mh, scale, ln_fast(safe)) : -INFINITY;
    }
    if constexpr (kFused) {
      // The slice goes to LDS as [head][column], then out with one 16-byte
      // store per lane and 4 columns (below).  Every wavefront stores the
      // group's LSEs (the same bits), so each slice's count covers them; the
      // stores are device-scope (sc1): written through to the coherence point,
      // so the merging wavefront on another XCD reads them without any cache
      // writeback.
#pragma unroll
      for (int j = 0; j < P::kNBW; ++j) wsm[w * 128 * GP + h * P::kCols + 16 * j + qh] = acc[j][r] * inv;
      if (lse_lane)
        __hip_atomic_store(lse_out + row0 + int64_t(h) * splits, lv, __ATOMIC_RELAXED, kScope);
    } else {
#pragma unroll
      for (int j = 0; j < P::kNBW; ++j) dst[16 * j] = acc[j][r] * inv;
      if (lse_lane) lse_out[row0 + int64_t(h) * splits] = lv;
    }
  }
  if constexpr (kFused) {
    // Lane l stores chunk l (+64, ...): head c / (kCols/4), 4 columns, 16 bytes.
    constexpr int kChunks = P::kCols / 4;
    const float* stage = wsm + w * 128 * GP;
    const int64_t grow = int64_t(b) * Hq + kh * G;
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(partials + grow * splits * D, G * splits * D * 4);
    for (int ch = lane; ch < G * kChunks; ch += 64) {
      const int h = ch / kChunks, c4 = 4 * (ch % kChunks);
      const u32x4_t val = *reinterpret_cast<const u32x4_t*>(stage + h * P::kCols + c4);
      __builtin_amdgcn_raw_buffer_store_b128(val, rs, ((h * splits + p) * D + w * P::kCols + c4) * 4,
                                             0, kCoherentAux);
    }
    count_and_merge();
  }
}

// ------------------------------------------------------------- LSE merge
// One wavefront per (b, h) row and 64-column chunk (grid rows x D/64), one
// output element per lane, so a row's partials are read by D/64 CUs at once.
// Every wavefront computes the row's weights itself (the same arithmetic, so
// the same bits in every chunk) and broadcasts them with readlane.
// Every load is in flight at once: a wavefront can have at most 63 vector
// loads outstanding, so one 4-byte load per split and lane would wait a
// second round trip past about 60 splits.  Instead the 16 lanes of 16-lane
// row r load the 64 columns of split 4 i + r as 16-byte pieces, four splits
// per instruction (kMax / 4 instructions, zeros past the last split), and a
// 4 x 4 transpose across the rows (v_permlane32_swap, then
// v_permlane16_swap) leaves lane 16 r + j with column 4 j + r of splits
// 4 i .. 4 i + 3.  The row's LSEs are loaded first, so the weights are
// computed while the partials arrive.  The chain acc = fma(w_p, partial_p,
// acc) runs over p = 0 .. kMax - 1 in order (matched_splitkv.py:121-126), kMax
// the split count rounded up to a multiple of 16; the terms past the last
// split are fma(0, 0, acc), which changes nothing but a -0 into +0.  The
// result is the same as a chain over 64 terms (128 past 64 splits) would give,
// the first form of this kernel: such a chain ends with zero terms unless the
// split count is 64 or 128, so a final acc + 0 stands in for them.
template <int D, int kMax>
__global__ void __launch_bounds__(64)
lse_merge_kernel(const float* __restrict__ partials, const float* __restrict__ lse,
                 uint16_t* __restrict__ out, int splits, int lanes) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const int c0 = blockIdx.y * 64;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(partials + row * splits * D, splits * D * 4);
  float la, lc;
  lse_load<0>(lse + row * splits, splits * 4, lane, la, lc);
  __builtin_amdgcn_sched_barrier(0);
  const int r = lane >> 4, j = lane & 15;
  float x[kMax / 4][4];
#pragma unroll
  for (int i = 0; i < kMax / 4; ++i)
    buffer_load_f32<4, 0>(rs, ((4 * i + r) * D + c0 + 4 * j) * 4, x[i]);
  __builtin_amdgcn_sched_barrier(0);
  float w0 = 0.f, w1 = 0.f;
  lse_weights_of(la, lc, splits, lanes, lane, w0, w1);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < kMax / 4; ++i) {
    // x[i][e] of row r is column 4 j + e of split 4 i + r; swap the row and
    // element bits, bit 1 (rows 0-1 <-> 2-3) then bit 0 (even <-> odd rows).
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[i][e]),
                                                      __float_as_uint(x[i][e + 2]), false, false);
      x[i][e] = __uint_as_float(t[0]);
      x[i][e + 2] = __uint_as_float(t[1]);
    }
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[i][e]),
                                                      __float_as_uint(x[i][e + 1]), false, false);
      x[i][e] = __uint_as_float(t[0]);
      x[i][e + 1] = __uint_as_float(t[1]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = fmaf(wave_weight(w0, w1, 4 * i + k), x[i][k], acc);
  }
  if (splits % 64 != 0) acc = acc + 0.f;
  out[row * D + c0 + 4 * j + r] = uint16_t(bf16_bits(acc));
}

// ------------------------------------------------------------ m/l/acc merge
// The merge of the fixed-split protocol (kernels.py:83-100): M = max_p m_p
// (-inf -> 0), f_p = exp(m_p - M), out = sum_p f_p acc_p / sum_p f_p l_p (a
// zero total divides by 1).  Up to 128 partitions: one wavefront per (b, h)
// row and 64 E columns (grid rows x D / (64 E)), E consecutive columns per
// lane; E = 1 spreads a row over D / 64 CUs when there are few rows.  Lane j
// loads m and l of partitions j and j + 64; every accumulator load of a batch
// of kBatch partitions is issued before the factors are computed
// (merge_splits), the total is an xor-butterfly sum over the lanes, and
// acc = fma(f_p, acc_p, acc) runs in partition order.  Loads past the row read
// zero and carry f = 0, so neither E nor kBatch changes the result's bits.
template <int E, int kBatch>
__global__ void __launch_bounds__(64)
ml_merge_kernel(const float* __restrict__ maxima, const float* __restrict__ denoms,
                const float* __restrict__ accums, uint16_t* __restrict__ out, int parts, int D) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const int col = (blockIdx.y * 64 + lane) * E;
  const __amdgpu_buffer_rsrc_t rm = buffer_rsrc(maxima + row * parts, parts * 4);
  const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(denoms + row * parts, parts * 4);
  float m0[1], m1[1], l0[1], l1[1];
  buffer_load_f32<1, 0>(rm, lane * 4, m0);
  buffer_load_f32<1, 0>(rm, (lane + 64) * 4, m1);
  buffer_load_f32<1, 0>(rl, lane * 4, l0);
  buffer_load_f32<1, 0>(rl, (lane + 64) * 4, l1);
  float f0 = 0.f, f1 = 0.f, inv = 1.f, acc[E];
  merge_splits<E, 0, kBatch>(
      accums + row * parts * D, D, col, parts,
      [&] {
        const float v0 = lane < parts ? m0[0] : -INFINITY;
        const float v1 = lane + 64 < parts ? m1[0] : -INFINITY;
        float mx = wave_max(fmaxf(v0, v1));
        if (mx == -INFINITY) mx = 0.f;  // all partitions empty
        f0 = exp_fast(v0 - mx);
        f1 = exp_fast(v1 - mx);
        const float total = wave_sum(fmaf(l1[0], f1, l0[0] * f0));
        inv = 1.f / (total > 0.f ? total : 1.f);
      },
      [&](int s0, int j) { return wave_weight(f0, f1, s0 + j); }, acc);
#pragma unroll
  for (int e = 0; e < E; ++e) out[row * D + col + e] = uint16_t(bf16_bits(acc[e] * inv));
}

// The same merge for more than 128 partitions: one wavefront per row, lane j
// owning columns VEC j .. VEC j + VEC - 1, partitions in order.
template <int VEC>
__global__ void __launch_bounds__(64)
ml_merge_loop_kernel(const float* __restrict__ maxima, const float* __restrict__ denoms,
                     const float* __restrict__ accums, uint16_t* __restrict__ out, int parts) {
  constexpr int D = VEC * 64;
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const float* mrow = maxima + int64_t(row) * parts;
  const float* lrow = denoms + int64_t(row) * parts;
  float mx = -INFINITY;
  for (int p = lane; p < parts; p += 64) mx = fmaxf(mx, mrow[p]);
  mx = wave_max(mx);
  if (mx == -INFINITY) mx = 0.f;  // all partitions empty
  float total = 0.f, acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  const float* arow = accums + int64_t(row) * parts * D + lane * VEC;
  for (int p = 0; p < parts; ++p) {
    const float f = exp_fast(mrow[p] - mx);
    total += lrow[p] * f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = fmaf(arow[int64_t(p) * D + e], f, acc[e]);
  }
  const float inv = 1.f / (total > 0.f ? total : 1.f);
  uint16_t* dst = out + int64_t(row) * D + lane * VEC;
#pragma unroll
  for (int e = 0; e < VEC; ++e) dst[e] = uint16_t(bf16_bits(acc[e] * inv));
}

// ----------------------------------------------------- online m/l/acc merge
// The merge of pd_split_decode's one-workgroup-per-partition grid: the
// fixed-split merge (kernels.py:83-100) in the online form of ml_step (pd_device.h): partitions p = P - 1 down to 0, empty ones
// skipped, a running maximum, out = acc / total (a zero total divides by 1).
// Up to 128 partitions: one wavefront per (b, h) row and 64 E columns (grid
// rows x D / (64 E)), E consecutive columns per lane; E = 1 spreads a row over
// D / 64 CUs when there are few rows.  The accumulator loads of kBatch
// partitions (from the top) are issued first; lane j loads m and l of
// partitions j and j + 64 and computes their steps' factors (ml_steps_of)
// while they arrive.  The chain acc = fma(acc_p, b, acc * a) then takes each
// partition's factors with v_readlane, eight partitions at a time.  An empty
// partition's a = 1, b = 0 over its zero accumulators (as the partition
// kernels write them) leave acc and total unchanged, as skipping it does, and
// so do the padding steps past partition 0 over zero loads: the chain has no
// branch.  Neither E nor kBatch changes the result's bits, and the walk's
// in-kernel merge (cols_loader_kernel, kSplit) gives the same bits.
template <int E, int kBatch>
__global__ void __launch_bounds__(64)
ml_online_merge_kernel(const float* __restrict__ maxima, const float* __restrict__ denoms,
                const float* __restrict__ accums, uint16_t* __restrict__ out, int parts, int D) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const int col = (blockIdx.y * 64 + lane) * E;
  const __amdgpu_buffer_rsrc_t rm = buffer_rsrc(maxima + row * parts, parts * 4);
  const __amdgpu_buffer_rsrc_t rl = buffer_rsrc(denoms + row * parts, parts * 4);
  const int bytes = parts * D * 4;
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(accums + row * parts * D, bytes);
  float m0[1], m1[1], l0[1], l1[1];
  buffer_load_f32<1, 0>(rm, lane * 4, m0);
  buffer_load_f32<1, 0>(rm, (lane + 64) * 4, m1);
  buffer_load_f32<1, 0>(rl, lane * 4, l0);
  buffer_load_f32<1, 0>(rl, (lane + 64) * 4, l1);
  float x[kBatch][E];
  auto load = [&](int top) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int p = top - 1 - j;
      buffer_load_f32<E, 0>(ra, p >= 0 ? (p * D + col) * 4 : bytes, x[j]);
    }
  };
  load(parts);
  __builtin_amdgcn_sched_barrier(0);
  MlStep s0, s1;
  ml_steps_of(m0[0], m1[0], parts, lane, s0, s1);
  // Loads past the row read zero, so the l of a padding partition is 0.
  float acc[E], total = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  // A do-while (parts >= 1): a loop guard in front would let the compiler
  // sink the first batch's loads past the factors' computation.
  int top = parts;
  do {
    if (top != parts) load(top);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (j % 8 == 0) __builtin_amdgcn_sched_barrier(0);  // bounds the readlanes in flight
      const int p = top - 1 - j;
      const int src = p & 63;
      const bool upper = p >= 64;
      // Read unconditionally, then select: a lane read under a branch would
      // need the branch.
      const float ra = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, upper ? s1.a : s0.a), src));
      const float rb = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, upper ? s1.b : s0.b), src));
      const float rl_ = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, upper ? l1[0] : l0[0]), src));
      const float a = p < 0 ? 1.f : ra, bp = p < 0 ? 0.f : rb, lp = p < 0 ? 0.f : rl_;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = fmaf(x[j][e], bp, acc[e] * a);
      total = fmaf(lp, bp, total * a);
    }
    top -= kBatch;
  } while (top > 0);
  const float inv = 1.f / (total > 0.f ? total : 1.f);
#pragma unroll
  for (int e = 0; e < E; ++e) out[row * D + col + e] = uint16_t(bf16_bits(acc[e] * inv));
}

// The same merge for more than 128 partitions: one wavefront per row, lane j
// owning columns VEC j .. VEC j + VEC - 1, ml_step in partition order from
// the last.
template <int VEC>
__global__ void __launch_bounds__(64)
ml_online_merge_loop_kernel(const float* __restrict__ maxima, const float* __restrict__ denoms,
                     const float* __restrict__ accums, uint16_t* __restrict__ out, int parts) {
  constexpr int D = VEC * 64;
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const float* mrow = maxima + int64_t(row) * parts;
  const float* lrow = denoms + int64_t(row) * parts;
  float M = -INFINITY, total = 0.f, acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  const float* arow = accums + int64_t(row) * parts * D + lane * VEC;
  for (int p = parts - 1; p >= 0; --p) {
    const MlStep st = ml_step(mrow[p], M);
    if (!st.live) continue;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = fmaf(arow[int64_t(p) * D + e], st.b, acc[e] * st.a);
    total = fmaf(lrow[p], st.b, total * st.a);
  }
  const float inv = 1.f / (total > 0.f ? total : 1.f);
  uint16_t* dst = out + int64_t(row) * D + lane * VEC;
#pragma unroll
  for (int e = 0; e < VEC; ++e) dst[e] = uint16_t(bf16_bits(acc[e] * inv));
}

// --------------------------------------------------------------- launchers

int launch_status(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return pd::fail(PD_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(err));
  return PD_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_qkv(const void* q, int64_t qsb, int64_t qsh, const void* k, const void* v,
              const int32_t* table, int32_t width, const int32_t* lengths, int32_t batch,
              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0)
    return pd::fail(PD_EINVAL, "batch and head counts must be positive");
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (num_heads % num_kv_heads)
    return pd::fail(PD_EINVAL, "query heads must be divisible by KV heads");
  if (!q || !k || !v || !table || !lengths) return pd::fail(PD_EINVAL, "null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (qsb & 7) || (qsh & 7) || qsb < 0 ||
      qsh < 0)
    return pd::fail(PD_EINVAL,
                    "Q/K/V rows must be 16-byte aligned (strides multiples of 8 elements)");
  if (qsb >= (int64_t(1) << 31) || qsh >= (int64_t(1) << 31))
    return pd::fail(PD_EINVAL, "Q strides must stay below 2^31 elements");
  if (int64_t(num_kv_heads) * head_dim * 512 >= (int64_t(1) << 31))
    return pd::fail(PD_EINVAL, "a 256-slot page of one KV tensor must stay below 2 GiB");
  if (width < 1 || width >= (1 << 22))
    return pd::fail(PD_EINVAL, "table width must be in [1, 2^22)");
  return PD_OK;
}

// Kernel argument order puts what the first memory accesses need (table row,
// length, query rows) first: those arguments fit the SGPRs the hardware fills
// before the first instruction (kernarg preloading), so the first loads do
// not wait for a kernel-argument fetch.  Strides are int32 (checked).
struct PartitionArgs {
  const uint16_t* q;
  int qsb, qsh;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* table;
  int tsb;
  int width;
  const int32_t* lengths;
  float* partials;
  float* lse;
  int* counters;
  uint16_t* out;
  float* maxima;
  int Hq, Hkv, G, hs, splits, T;
  float scale, c;
  int order = -1;  // batch order of the multi-tile kernels (batch_order)
  int wf = 1;      // partitions per workgroup of the walks (kSplit, kMatchedWalk)
};

// Compute units of the current device, queried once per device.
int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 0;
  }
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      n = -1;
    }
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// `order` of ordered_sequence (pd_device.h) for a multi-tile launch over
// `grid` = (splits, kv heads x slices, batch), one workgroup per CU:
// * 0 (longest first) for two to four rounds of workgroups;
// * -1 (sequence z) when every workgroup has a CU to itself, the batch has one
//   sequence or more than kMaxOrderedBatch, the CU count is unknown, or the
//   grid runs more than four rounds.  There the ranking's extra round trip at
//   the start of every workgroup costs more than the order gains: with 8192
//   mostly short workgroups (batch 128, lengths up to 4096, D 64, 16 kv heads,
//   4 fixed partitions, two workgroups per CU) it took the call from 228 to
//   275 us, and sorting the batch on the host gained nothing there.
int batch_order(dim3 grid) {
  const int B = int(grid.z);
  if (B < 2 || B > kMaxOrderedBatch) return -1;
  const int cus = device_cu_count();
  if (cus <= 0) return -1;
  const int64_t n = int64_t(grid.x) * grid.y * B;
  return n <= cus || n > 4 * int64_t(cus) ? -1 : 0;
}

template <int D, bool kFused>
void launch_tile_d(int gp, dim3 grid, hipStream_t stream, const PartitionArgs& a) {
#define PD_LAUNCH_TILE(GPV)                                                                    \
  hipLaunchKernelGGL((matched_tile_kernel<D, GPV, kFused>), grid, dim3(kThreads), 0, stream,    \
                     a.table, a.lengths, a.q, a.tsb, a.width, a.qsb, a.qsh, a.G, a.Hq, a.splits, \
                     a.k, a.v, a.partials, a.lse, a.Hkv, a.scale, a.c, a.counters, a.out)
  switch (gp) {
    case 1: PD_LAUNCH_TILE(1); break;
    case 2: PD_LAUNCH_TILE(2); break;
    case 4: PD_LAUNCH_TILE(4); break;
    case 8: PD_LAUNCH_TILE(8); break;
    default: PD_LAUNCH_TILE(16); break;
  }
#undef PD_LAUNCH_TILE
}

// The multi-tile partition with loader wavefronts (cols_loader_kernel).
template <int D, bool kFused, int kMode, int kHeads = 1>
void launch_cols_loader(int gp, dim3 grid, hipStream_t stream, const PartitionArgs& a) {
#define PD_LAUNCH_LOADER(GPV)                                                                  \
  hipLaunchKernelGGL((cols_loader_kernel<D, GPV, kFused, kMode, kHeads>), grid, dim3(2 * kThreads), 0, \
                     stream, a.table, a.lengths, a.q, a.tsb, a.width, a.order, a.T, a.qsb,     \
                     a.qsh, a.G, a.hs, a.Hq, a.k, a.v, a.partials, a.lse, a.counters, a.out,   \
                     a.maxima, a.Hkv, a.splits, a.scale, a.c, a.wf)
  switch (gp) {
    case 1: PD_LAUNCH_LOADER(1); break;
    case 2: PD_LAUNCH_LOADER(2); break;
    case 4: PD_LAUNCH_LOADER(4); break;
    case 8: PD_LAUNCH_LOADER(8); break;
    default: PD_LAUNCH_LOADER(16); break;
  }
#undef PD_LAUNCH_LOADER
}

// Longest split (in tiles) that the matched protocol walks several of per
// workgroup (partition_entry).
constexpr int kWalkMaxSplitTiles = 5;

int padded_group(int g) {
  int gp = 1;
  while (gp < g) gp <<= 1;
  return gp;
}

// A matched plan of one split longer than a tile: the partition kernel
// (cols_loader_kernel) writes the output itself and no merge runs.
bool one_split_direct(int32_t splits, int32_t tokens_per_split, int32_t tile_tokens) {
  return splits == 1 && tokens_per_split != tile_tokens;
}

// Validation and dispatch shared by pd_partition (fused = false) and
// pd_matched_decode (fused = true, or fused = false with an output for a plan
// of one split).
int partition_entry(const char* what, bool fused, const void* q, int64_t qsb, int64_t qsh,
                    const void* k, const void* v, const int32_t* table, int64_t tsb,
                    int32_t width, const int32_t* lengths, float* partials, float* lse,
                    int32_t* counters,
                    void* out, int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                    int32_t head_dim, int32_t splits, int32_t tokens_per_split,
                    int32_t tile_tokens, double scale, pd_stream_t stream) {
  pd::clear_error();
  if (int st = check_qkv(q, qsb, qsh, k, v, table, width, lengths, batch, num_heads,
                         num_kv_heads, head_dim))
    return st;
  const int G = num_heads / num_kv_heads;
  if (G > 16)
    return pd::fail(PD_EINVAL, "matched split-KV requires at most 16 query heads per KV head");
  if (splits < 1 || splits > 128) return pd::fail(PD_EINVAL, "splits must be in [1,128]");
  if (tile_tokens != 16384 / head_dim)
    return pd::fail(PD_EINVAL, "tile_tokens must be %d for head_dim %d", 16384 / head_dim,
                    head_dim);
  if (tokens_per_split <= 0 || tokens_per_split % tile_tokens)
    return pd::fail(PD_EINVAL, "tokens_per_split must be a positive multiple of tile_tokens");
  if (int64_t(splits) * tokens_per_split >= (int64_t(1) << 31))
    return pd::fail(PD_EINVAL, "splits * tokens_per_split must stay below 2^31");
  if (!partials || !lse || (fused && (!counters || !out)))
    return pd::fail(PD_EINVAL, "invalid matched workspace");
  if (!(scale > 0.0) || !std::isfinite(scale))
    return pd::fail(PD_EINVAL, "positive finite scale required");
  if (batch > 65535 || num_kv_heads > 65535)
    return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  if (tsb < 0 || tsb >= (int64_t(1) << 31))
    return pd::fail(PD_EINVAL, "block table row stride must be in [0, 2^31)");
  // Without the fused merge, `out` is written only by a plan of one split of
  // more than one tile (its merge is the identity, one_split_direct).
  if (!fused && !one_split_direct(splits, tokens_per_split, tile_tokens)) out = nullptr;
  PartitionArgs a{static_cast<const uint16_t*>(q), int(qsb), int(qsh),
                  static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), table,
                  int(tsb), width, lengths, partials, lse,
                  counters, static_cast<uint16_t*>(out), nullptr, num_heads, num_kv_heads, G, 1,
                  splits,
                  tokens_per_split, float(scale),
                  float(scale * 1.4426950408889634)};  // SCALE_LOG2 (matched_splitkv.py:363)
  const dim3 grid(splits, num_kv_heads, batch);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int gp = padded_group(G);
  if (tokens_per_split == tile_tokens) {
    switch (head_dim * 2 + (fused ? 1 : 0)) {
      case 128: launch_tile_d<64, false>(gp, grid, st, a); break;
      case 129: launch_tile_d<64, true>(gp, grid, st, a); break;
      case 256: launch_tile_d<128, false>(gp, grid, st, a); break;
      case 257: launch_tile_d<128, true>(gp, grid, st, a); break;
      case 512: launch_tile_d<256, false>(gp, grid, st, a); break;
      default: launch_tile_d<256, true>(gp, grid, st, a); break;
    }
    return launch_status(what);
  }
  // Plans of short splits with more workgroups than CUs walk wf consecutive
  // splits per workgroup (kMatchedWalk), so that one resident round of
  // workgroups runs them; every split keeps its bits.  A workgroup's start
  // (table, query and first tiles in flight) then runs once instead of wf
  // times, but each split before the last is stored while the K / V stream
  // runs, which costs a few microseconds when every CU streams.  Paired A/B
  // at Hq 16 / Hkv 4 / D 256 (walk against one workgroup per split): splits
  // of 2 to 5 tiles 1.2-19% faster (ctx 8192 x 2 sequences, 2064 x 8 and x 16,
  // 32768, 8192 x 4); splits of 9 or 10 tiles 1-13% slower (4096 x 16,
  // 8192 x 8, 16384 x 4, 32768 x 2, 65536), with one exception (2064 x 32,
  // whose last splits are short).
  const int cus = device_cu_count();
  const int64_t wgs = int64_t(splits) * num_kv_heads * batch;
  if (!fused && cus > 0 && splits > 1 && wgs > cus &&
      tokens_per_split <= kWalkMaxSplitTiles * tile_tokens) {
    a.wf = int(std::min<int64_t>((wgs + cus - 1) / cus, splits));
    const dim3 wgrid((splits + a.wf - 1) / a.wf, num_kv_heads, batch);
    a.order = batch_order(wgrid);
    switch (head_dim) {
      case 64: launch_cols_loader<64, false, kMatchedWalk>(gp, wgrid, st, a); break;
      case 128: launch_cols_loader<128, false, kMatchedWalk>(gp, wgrid, st, a); break;
      default: launch_cols_loader<256, false, kMatchedWalk>(gp, wgrid, st, a); break;
    }
    return launch_status(what);
  }
  a.order = batch_order(grid);
  switch (head_dim * 2 + (fused ? 1 : 0)) {
    case 128: launch_cols_loader<64, false, kMatched>(gp, grid, st, a); break;
    case 129: launch_cols_loader<64, true, kMatched>(gp, grid, st, a); break;
    case 256: launch_cols_loader<128, false, kMatched>(gp, grid, st, a); break;
    case 257: launch_cols_loader<128, true, kMatched>(gp, grid, st, a); break;
    case 512: launch_cols_loader<256, false, kMatched>(gp, grid, st, a); break;
    default: launch_cols_loader<256, true, kMatched>(gp, grid, st, a); break;
  }
  return launch_status(what);
}

}  // namespace

extern "C" int pd_partition(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            const void* k, const void* v, const int32_t* table,
                            int64_t table_stride_b, int32_t table_width, const int32_t* lengths,
                            float* partials, float* lse, int32_t batch, int32_t num_heads,
                            int32_t num_kv_heads, int32_t head_dim, int32_t splits,
                            int32_t tokens_per_split, int32_t tile_tokens, double scale,
                            pd_stream_t stream) {
  return partition_entry("pd_partition", false, q, q_stride_b, q_stride_h, k, v, table,
                         table_stride_b, table_width, lengths, partials, lse, nullptr, nullptr,
                         batch,
                         num_heads, num_kv_heads, head_dim, splits, tokens_per_split,
                         tile_tokens, scale, stream);
}

namespace {
int merge_entry(const char* what, const float* partials, const float* lse, void* out,
                int32_t batch, int32_t num_heads, int32_t head_dim, int32_t splits,
                int32_t lse_lanes, pd_stream_t stream);
}  // namespace

extern "C" int pd_matched_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                 const void* k, const void* v, const int32_t* table,
                                 int64_t table_stride_b, int32_t table_width,
                                 const int32_t* lengths, float* partials, float* lse,
                                 int32_t* counters, void* out,
                                 int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t splits, int32_t tokens_per_split,
                                 int32_t tile_tokens, double scale, pd_stream_t stream) {
  if (counters != nullptr)
    return partition_entry("pd_matched_decode", true, q, q_stride_b, q_stride_h, k, v, table,
                           table_stride_b, table_width, lengths, partials, lse, counters, out,
                           batch, num_heads, num_kv_heads, head_dim, splits, tokens_per_split,
                           tile_tokens, scale, stream);
  // Without counters: the partition and the LSE merge as two launches, or the
  // partition alone, writing the output, for a plan of one split.
  pd::clear_error();
  if (!out) return pd::fail(PD_EINVAL, "invalid matched workspace");
  if (int st = partition_entry("pd_matched_decode", false, q, q_stride_b, q_stride_h, k, v,
                               table, table_stride_b, table_width, lengths, partials, lse,
                               nullptr, out, batch, num_heads, num_kv_heads, head_dim, splits,
                               tokens_per_split, tile_tokens, scale, stream))
    return st;
  if (one_split_direct(splits, tokens_per_split, tile_tokens)) return PD_OK;
  return merge_entry("pd_matched_decode", partials, lse, out, batch, num_heads, head_dim,
                     splits, plan_lse_lanes(splits, head_dim), stream);
}

namespace {

// Validation and launch of lse_merge_kernel, shared by pd_lse_merge and
// pd_matched_decode_noalloc.
int merge_entry(const char* what, const float* partials, const float* lse, void* out,
                int32_t batch, int32_t num_heads, int32_t head_dim, int32_t splits,
                int32_t lse_lanes, pd_stream_t stream) {
  if (batch <= 0 || num_heads <= 0) return pd::fail(PD_EINVAL, "batch and heads must be positive");
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (splits < 1 || splits > 128) return pd::fail(PD_EINVAL, "splits must be in [1,128]");
  if (lse_lanes < 1 || lse_lanes > 64 || (lse_lanes & (lse_lanes - 1)))
    return pd::fail(PD_EINVAL, "lse_lanes must be a power of two in [1, 64]");
  if (lse_lanes > 1 && lse_lanes / 2 >= splits)
    return pd::fail(PD_EINVAL, "lse_lanes must not exceed the next power of two of splits");
  if (!partials || !lse || !out) return pd::fail(PD_EINVAL, "null tensor pointer");
  if (!aligned16(partials)) return pd::fail(PD_EINVAL, "partials must be 16-byte aligned");
  const int64_t rows = int64_t(batch) * num_heads;
  if (rows > 0x7fffffff) return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto* o = static_cast<uint16_t*>(out);
  const dim3 grid(unsigned(rows), head_dim / 64);
#define PD_LAUNCH_MERGE_K(DV, KM)                                                              \
  case KM / 16:                                                                                \
    hipLaunchKernelGGL((lse_merge_kernel<DV, KM>), grid, dim3(64), 0, st, partials, lse, o,    \
                       splits, lse_lanes);                                                     \
    break
#define PD_LAUNCH_MERGE(DV)                                                                    \
  switch ((splits + 15) / 16) {                                                                \
    PD_LAUNCH_MERGE_K(DV, 16); PD_LAUNCH_MERGE_K(DV, 32); PD_LAUNCH_MERGE_K(DV, 48);           \
    PD_LAUNCH_MERGE_K(DV, 64); PD_LAUNCH_MERGE_K(DV, 80); PD_LAUNCH_MERGE_K(DV, 96);           \
    PD_LAUNCH_MERGE_K(DV, 112); default: PD_LAUNCH_MERGE_K(DV, 128);                           \
  }
  switch (head_dim) {
    case 64: PD_LAUNCH_MERGE(64); break;
    case 128: PD_LAUNCH_MERGE(128); break;
    default: PD_LAUNCH_MERGE(256); break;
  }
#undef PD_LAUNCH_MERGE
#undef PD_LAUNCH_MERGE_K
  return launch_status(what);
}

}  // namespace

extern "C" int pd_lse_merge(const float* partials, const float* lse, void* out, int32_t batch,
                            int32_t num_heads, int32_t head_dim, int32_t splits,
                            int32_t lse_lanes, pd_stream_t stream) {
  pd::clear_error();
  return merge_entry("pd_lse_merge", partials, lse, out, batch, num_heads, head_dim, splits,
                     lse_lanes, stream);
}

// ------------------------------------------------ allocation-free decode
// The split workspace of pd_matched_decode_noalloc lives in this file-scope
// device array: partials f32 [batch, num_heads, splits, head_dim] from byte 0,
// then lse f32 [batch, num_heads, splits] from the next 256-byte boundary.
// Every GPU the library runs on holds its own copy until the process ends.  In
// host code `pd_scratch` names a host-side stand-in, never the device memory:
// the device address comes from hipGetSymbolAddress, once per device, with that
// device current.
static __device__ __align__(256) unsigned char pd_scratch[PD_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

// Device address of pd_scratch on the current device, looked up on the first
// call per device; nullptr (with pd_last_error set) if the lookup fails.
void* scratch_address() {
  static std::atomic<void*> cache[kMaxDevices];
  static std::mutex mu;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    pd::fail(PD_ELAUNCH, "no current HIP device (or device index past %d)", kMaxDevices - 1);
    return nullptr;
  }
  void* ptr = cache[dev].load(std::memory_order_acquire);
  if (ptr) return ptr;
  std::lock_guard<std::mutex> lock(mu);
  ptr = cache[dev].load(std::memory_order_relaxed);
  if (!ptr) {
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(pd_scratch));
    if (err != hipSuccess || !ptr) {
      (void)hipGetLastError();
      pd::fail(PD_ELAUNCH, "hipGetSymbolAddress(pd_scratch) failed on device %d: %s", dev,
               hipGetErrorString(err));
      return nullptr;
    }
    cache[dev].store(ptr, std::memory_order_release);
  }
  return ptr;
}

}  // namespace

extern "C" int pd_matched_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                         const void* k, const void* v, const int32_t* table,
                                         int64_t table_stride_b, int32_t table_width,
                                         const int32_t* lengths, void* out, int32_t batch,
                                         int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t splits,
                                         int32_t tokens_per_split, int32_t tile_tokens,
                                         double scale, pd_stream_t stream) {
  pd::clear_error();
  if (batch <= 0 || num_heads <= 0 || splits < 1 || splits > 128 ||
      !pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "batch, heads, head_dim (64/128/256) and splits (1..128) must "
                               "be valid");
  const int64_t rows = int64_t(batch) * num_heads * splits;
  const int64_t lse_offset = (rows * head_dim * 4 + 255) / 256 * 256;
  const int64_t need = lse_offset + rows * 4;
  if (need > int64_t(PD_NOALLOC_SCRATCH_BYTES))
    return pd::fail(PD_EINVAL,
                    "split workspace of %lld bytes (batch * num_heads * splits * (head_dim + 1) "
                    "floats) exceeds the %lld-byte static scratch of pd_matched_decode_noalloc",
                    static_cast<long long>(need),
                    static_cast<long long>(PD_NOALLOC_SCRATCH_BYTES));
  if (!out) return pd::fail(PD_EINVAL, "invalid output buffer");
  auto* base = static_cast<unsigned char*>(scratch_address());
  if (!base) return PD_ELAUNCH;
  auto* partials = reinterpret_cast<float*>(base);
  auto* lse = reinterpret_cast<float*>(base + lse_offset);
  if (int st = partition_entry("pd_matched_decode_noalloc", false, q, q_stride_b, q_stride_h, k,
                               v, table, table_stride_b, table_width, lengths, partials, lse,
                               nullptr, out, batch, num_heads, num_kv_heads, head_dim,
                               splits, tokens_per_split, tile_tokens, scale, stream))
    return st;
  if (one_split_direct(splits, tokens_per_split, tile_tokens)) return PD_OK;
  return merge_entry("pd_matched_decode_noalloc", partials, lse, out, batch, num_heads,
                     head_dim, splits, plan_lse_lanes(splits, head_dim), stream);
}

namespace {

// The m/l/acc merge over `rows` (b, h) rows, up to 128 partitions in one
// wavefront per row and 64 E columns, more in one wavefront per row:
// ml_merge_kernel / ml_merge_loop_kernel (the reference's order), or with
// kOnline their online forms (pd_split_decode's order).  Arguments checked by
// the caller.
template <bool kOnline>
void launch_ml_merge(const float* maxima, const float* denoms, const float* accums, uint16_t* o,
                     int64_t rows, int head_dim, int partitions, hipStream_t st) {
  if (partitions <= 128) {
    // One wavefront per row (E = D / 64 columns per lane, 16-byte aligned
    // accumulators) once the rows alone give 2048 wavefronts or more; otherwise a
    // row's 64-column chunks on as many wavefronts.  Load batches of 4 to 48
    // partitions (at most 16 of E > 1 columns).
    const int E = rows >= 2048 && aligned16(accums) ? head_dim / 64 : 1;
    int batch = 4;
    while (batch < partitions && batch < (E == 1 ? 48 : 16)) batch = batch < 32 ? 2 * batch : 48;
    const dim3 grid(unsigned(rows), head_dim / (64 * E));
#define PD_LAUNCH_ML(EV, KB)                                                                   \
  if (kOnline)                                                                                 \
    hipLaunchKernelGGL((ml_online_merge_kernel<EV, KB>), grid, dim3(64), 0, st, maxima, denoms,  \
                       accums, o, partitions, head_dim);                                       \
  else                                                                                         \
    hipLaunchKernelGGL((ml_merge_kernel<EV, KB>), grid, dim3(64), 0, st, maxima, denoms, accums, \
                       o, partitions, head_dim)
    switch (E * 100 + batch) {
      case 104: PD_LAUNCH_ML(1, 4); break;
      case 108: PD_LAUNCH_ML(1, 8); break;
      case 116: PD_LAUNCH_ML(1, 16); break;
      case 132: PD_LAUNCH_ML(1, 32); break;
      case 148: PD_LAUNCH_ML(1, 48); break;
      case 204: PD_LAUNCH_ML(2, 4); break;
      case 208: PD_LAUNCH_ML(2, 8); break;
      case 216: PD_LAUNCH_ML(2, 16); break;
      case 404: PD_LAUNCH_ML(4, 4); break;
      case 408: PD_LAUNCH_ML(4, 8); break;
      default: PD_LAUNCH_ML(4, 16); break;
    }
#undef PD_LAUNCH_ML
    return;
  }
  switch (head_dim) {
    case 64:
      if (kOnline)
        hipLaunchKernelGGL(ml_online_merge_loop_kernel<1>, dim3(rows), dim3(64), 0, st, maxima,
                           denoms, accums, o, partitions);
      else
        hipLaunchKernelGGL(ml_merge_loop_kernel<1>, dim3(rows), dim3(64), 0, st, maxima, denoms,
                           accums, o, partitions);
      break;
    case 128:
      if (kOnline)
        hipLaunchKernelGGL(ml_online_merge_loop_kernel<2>, dim3(rows), dim3(64), 0, st, maxima,
                           denoms, accums, o, partitions);
      else
        hipLaunchKernelGGL(ml_merge_loop_kernel<2>, dim3(rows), dim3(64), 0, st, maxima, denoms,
                           accums, o, partitions);
      break;
    default:
      if (kOnline)
        hipLaunchKernelGGL(ml_online_merge_loop_kernel<4>, dim3(rows), dim3(64), 0, st, maxima,
                           denoms, accums, o, partitions);
      else
        hipLaunchKernelGGL(ml_merge_loop_kernel<4>, dim3(rows), dim3(64), 0, st, maxima, denoms,
                           accums, o, partitions);
      break;
  }
}

// Whether pd_split_fixed runs one workgroup per partition: when the walks,
// one per (kv head group, sequence), leave CUs of the device idle and there is
// more than one partition.
bool per_partition_grid(int parts, int ygrid, int batch) {
  const int cus = device_cu_count();
  return parts > 1 && cus > 0 && int64_t(ygrid) * batch < cus;
}

// The base / fixed-split partition kernel for one protocol, head dim and
// kv-head grouping.
template <int kMode>
void launch_online_mode(int head_dim, int heads, int G, dim3 grid, hipStream_t st,
                        const PartitionArgs& a) {
  if (heads == 4) {
    launch_cols_loader<64, false, kMode, 4>(padded_group(4 * G), grid, st, a);
    return;
  }
  if (heads == 2) {
    launch_cols_loader<64, false, kMode, 2>(padded_group(2 * G), grid, st, a);
    return;
  }
  const int gp = padded_group(G < 16 ? G : 16);
  switch (head_dim) {
    case 64: launch_cols_loader<64, false, kMode>(gp, grid, st, a); break;
    case 128: launch_cols_loader<128, false, kMode>(gp, grid, st, a); break;
    default: launch_cols_loader<256, false, kMode>(gp, grid, st, a); break;
  }
}

// pd_base and pd_split_fixed: the partition kernel in its base / fixed-split
// protocol, one workgroup per (kv head [group or 16-head slice], sequence),
// or per (partition, kv head, sequence) for fixed splits at small grids.
template <bool kSplitMode>
int launch_online(const void* q, int64_t qsb, int64_t qsh, const void* k, const void* v,
                  const int32_t* table, int64_t tsb, int32_t width, const int32_t* lengths,
                  void* out,
                  float* maxima, float* denoms, float* accums, int32_t batch, int32_t num_heads,
                  int32_t num_kv_heads, int32_t head_dim, int32_t parts, int32_t part_size,
                  double scale, pd_stream_t stream, const char* what) {
  if (int st = check_qkv(q, qsb, qsh, k, v, table, width, lengths, batch, num_heads,
                         num_kv_heads, head_dim))
    return st;
  if (!std::isfinite(scale)) return pd::fail(PD_EINVAL, "scale must be finite");
  const int G = num_heads / num_kv_heads;
  const int hs = (G + 15) / 16;
  if (batch > 65535 || int64_t(num_kv_heads) * hs > 65535)
    return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  const int tile = 16384 / head_dim;
  if (kSplitMode) {
    if (batch > 0 && int64_t(batch) * num_heads > 0x7fffffff)
      return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
    if (parts < 1) return pd::fail(PD_EINVAL, "partitions must be positive");
    if (part_size <= 0 || part_size % tile)
      return pd::fail(PD_EINVAL, "partition_size must be a positive multiple of %d", tile);
    if (int64_t(parts) * part_size >= (int64_t(1) << 31))
      return pd::fail(PD_EINVAL, "partitions * partition_size must stay below 2^31");
    if (!maxima || !denoms || !accums)
      return pd::fail(PD_EINVAL, "invalid or missing preallocated split-K workspace");
    if (!aligned16(accums))
      return pd::fail(PD_EINVAL, "split-K accumulators must be 16-byte aligned");
  } else if (!out) {
    return pd::fail(PD_EINVAL, "invalid output buffer");
  }
  // The base protocol is one partition as long as the table: lengths never
  // exceed width * 256 (the contract of the live table width).
  const int T = kSplitMode ? part_size : width * 256;
  if (tsb < 0 || tsb >= (int64_t(1) << 31))
    return pd::fail(PD_EINVAL, "block table row stride must be in [0, 2^31)");
  PartitionArgs a{static_cast<const uint16_t*>(q), int(qsb), int(qsh),
                  static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), table,
                  int(tsb), width, lengths, accums, denoms,
                  nullptr, static_cast<uint16_t*>(out), maxima, num_heads, num_kv_heads, G, hs,
                  kSplitMode ? parts : 1, T, float(scale), float(scale * 1.4426950408889634)};
  // At D = 64 a workgroup serves four or two adjacent kv heads when their
  // query heads fit one 16-head group: a token's 128-byte rows of those heads
  // are one contiguous read.
  const int heads = head_dim != 64 ? 1 : pd::heads_per_workgroup(num_kv_heads, G);
  const int ygrid = pd::walk_grid_y(num_heads, num_kv_heads, head_dim);
  // The fixed-split protocol walks each sequence in one workgroup and writes
  // every partition of it (grid.x = 1), like the base protocol, when the walks
  // fill the CUs.  With fewer (kv head, sequence) walks than CUs, it runs one
  // workgroup per partition instead (the same bits), as the reference's
  // _split grid does (runtime.py:111-113).
  const bool per_part = kSplitMode && per_partition_grid(parts, ygrid, batch);
  const dim3 grid(per_part ? parts : 1, ygrid, batch);
  a.wf = kSplitMode ? parts : 1;  // the walk covers every partition
  a.order = batch_order(grid);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (per_part) {
    // One workgroup per partition; with an output, ml_online_merge_kernel
    // merges them after (the walk's in-kernel merge has the same arithmetic).
    a.out = nullptr;
    launch_online_mode<kSplitPart>(head_dim, heads, G, grid, st, a);
    if (int s = launch_status(what)) return s;
    if (out) {
      launch_ml_merge<true>(maxima, denoms, accums, static_cast<uint16_t*>(out),
                            int64_t(batch) * num_heads, head_dim, parts, st);
    }
  } else {
    launch_online_mode<kSplitMode ? kSplit : kBase>(head_dim, heads, G, grid, st, a);
  }
  return launch_status(what);
}

}  // namespace

extern "C" int pd_base(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                       const void* v, const int32_t* table, int64_t table_stride_b,
                       int32_t table_width, const int32_t* lengths, void* out, int32_t batch,
                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, double scale,
                       pd_stream_t stream) {
  pd::clear_error();
  return launch_online<false>(q, q_stride_b, q_stride_h, k, v, table, table_stride_b,
                              table_width, lengths,
                              out, nullptr, nullptr, nullptr, batch, num_heads, num_kv_heads,
                              head_dim, 1, 0, scale, stream, "pd_base");
}

extern "C" int pd_split_fixed(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                              const void* k, const void* v, const int32_t* table,
                              int64_t table_stride_b, int32_t table_width,
                              const int32_t* lengths, float* maxima,
                              float* denoms, float* accums, int32_t batch, int32_t num_heads,
                              int32_t num_kv_heads, int32_t head_dim, int32_t partitions,
                              int32_t partition_size, double scale, pd_stream_t stream) {
  pd::clear_error();
  return launch_online<true>(q, q_stride_b, q_stride_h, k, v, table, table_stride_b,
                             table_width, lengths,
                             nullptr, maxima, denoms, accums, batch, num_heads, num_kv_heads,
                             head_dim, partitions, partition_size, scale, stream,
                             "pd_split_fixed");
}

extern "C" int pd_ml_merge(const float* maxima, const float* denoms, const float* accums,
                           void* out, int32_t batch, int32_t num_heads, int32_t head_dim,
                           int32_t partitions, pd_stream_t stream) {
  pd::clear_error();
  if (batch <= 0 || num_heads <= 0) return pd::fail(PD_EINVAL, "batch and heads must be positive");
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (partitions < 1) return pd::fail(PD_EINVAL, "partitions must be positive");
  if (!maxima || !denoms || !accums || !out)
    return pd::fail(PD_EINVAL, "invalid or missing preallocated split-K workspace");
  const int64_t rows = int64_t(batch) * num_heads;
  if (rows > 0x7fffffff) return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  launch_ml_merge<false>(maxima, denoms, accums, static_cast<uint16_t*>(out), rows, head_dim,
                         partitions, reinterpret_cast<hipStream_t>(stream));
  return launch_status("pd_ml_merge");
}

extern "C" int pd_split_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                               const void* k, const void* v, const int32_t* table,
                               int64_t table_stride_b, int32_t table_width,
                               const int32_t* lengths, float* maxima, float* denoms,
                               float* accums, void* out, int32_t batch, int32_t num_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t partitions,
                               int32_t partition_size, double scale, pd_stream_t stream) {
  pd::clear_error();
  if (!out) return pd::fail(PD_EINVAL, "invalid output buffer");
  return launch_online<true>(q, q_stride_b, q_stride_h, k, v, table, table_stride_b,
                             table_width, lengths, out, maxima, denoms, accums, batch, num_heads,
                             num_kv_heads, head_dim, partitions, partition_size, scale, stream,
                             "pd_split_decode");
}

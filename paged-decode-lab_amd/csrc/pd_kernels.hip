// Paged decode attention kernels for MI355X (gfx950, CDNA4) and their C-ABI
// launchers.  See include/paged_decode.h for the tensor contract.
//
// Kernels
//   matched_partition  one 256-thread workgroup per (split, kv head, sequence):
//                      QK^T on MFMA (v_mfma_f32_16x16x32_bf16), FP32 online
//                      softmax over 16384/D-token tiles walked last-to-first,
//                      PV on v_dot2_f32_bf16 with bf16(p) shared through LDS,
//                      normalized FP32 partial + LSE out.
//   lse_merge          one D-thread workgroup per (sequence, query head):
//                      stable log-sum-exp merge of the split partials, bf16 out.
//   online_decode      one 256-thread workgroup per (sequence, query head
//                      [, fixed partition]): FP32 online softmax with fp32 p,
//                      either normalized bf16 out (base) or (m, l, acc) state.
//   ml_merge           one wavefront per (sequence, query head): merge of the
//                      (m, l, acc) states.
//
// Every kernel reads the sequence length and block table on the device and
// never needs host-side knowledge of tensor contents, so launches are
// graph-capturable and replay correctly with new lengths, pages and KV.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "pd_internal.h"

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;  // ln 2 rounded to float32
constexpr int kThreads = 256;

// ---------------------------------------------------------------- numerics
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// float32 -> bfloat16 bits, round to nearest even; NaN -> quiet NaN.
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Native gfx950 transcendental instructions (v_exp_f32 = 2^x, v_log_f32 =
// log2 x, v_rcp_f32 = 1/x); ln and e^x by change of base.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float ln_fast(float x) { return __builtin_amdgcn_logf(x) * kLn2; }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// a.lo*b.lo + a.hi*b.hi + c over bf16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
  return x;
}

__device__ __forceinline__ u32x4_t load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// Buffer resource (V#) over `bytes` bytes at `base`; word 3 is the gfx9-family
// raw-buffer format.  Loads at or past `bytes` return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// E consecutive floats at byte offset `off`; kCoherent sets the sc1 cache
// policy bit (device-scope coherent, so a line another XCD wrote is re-read).
// The builtins' results are bit-cast as whole vectors to float vectors before
// any element is read: reading elements of their integer vector results
// directly made this compiler emit a single dword load for the whole vector.
template <int E, bool kCoherent>
__device__ __forceinline__ void buffer_load_f32(__amdgpu_buffer_rsrc_t rsrc, int off,
                                                float (&x)[E]) {
  constexpr int aux = kCoherent ? 16 : 0;
  if constexpr (E == 1) {
    x[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, aux));
  } else if constexpr (E == 2) {
    const u32x2_t t = __builtin_amdgcn_raw_buffer_load_b64(rsrc, off, 0, aux);
    const floatx2_t f = __builtin_bit_cast(floatx2_t, t);
    x[0] = f.x;
    x[1] = f.y;
  } else {
    static_assert(E % 4 == 0, "vector width");
#pragma unroll
    for (int i = 0; i < E; i += 4) {
      const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 4 * i, 0, aux);
      const floatx4_t f = __builtin_bit_cast(floatx4_t, t);
      x[i] = f.x;
      x[i + 1] = f.y;
      x[i + 2] = f.z;
      x[i + 3] = f.w;
    }
  }
}

// ------------------------------------------------------ LSE merge arithmetic
// Shared by the standalone merge kernel and the fused decode so that both give
// bit-identical outputs.
//
// Merge weights of one (b, h) row, computed by one full wavefront: lane owns
// splits `lane` and `lane + 64` (splits <= 128).  M = max lse (-inf -> 0),
// S = sum exp(lse - M), L = ln S + M (+inf when S == 0), w_p = exp(lse_p - L)
// (matched_splitkv.py:107-120; an all-empty row gets w = 0 everywhere).  The
// two loads are unconditional buffer loads (zero past the row, replaced by
// -inf), so they issue without a branch and queue behind earlier loads.
template <bool kCoherent>
__device__ __forceinline__ void lse_weights(const float* __restrict__ lrow, int splits, int lane,
                                            float& w0, float& w1) {
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(lrow, splits * 4);
  float a[1], c[1];
  buffer_load_f32<1, kCoherent>(rsrc, lane * 4, a);
  buffer_load_f32<1, kCoherent>(rsrc, (lane + 64) * 4, c);
  const float v0 = lane < splits ? a[0] : -INFINITY;
  const float v1 = lane + 64 < splits ? c[0] : -INFINITY;
  float mx = wave_max(fmaxf(v0, v1));
  if (mx == -INFINITY) mx = 0.f;
  const float total = wave_sum(exp_fast(v0 - mx) + exp_fast(v1 - mx));
  const float logsum = total > 0.f ? ln_fast(total) + mx : INFINITY;
  w0 = exp_fast(v0 - logsum);
  w1 = exp_fast(v1 - logsum);
}

// acc[e] = fma(w_p, partial_p[e], acc[e]) for p = 0, 1, ..., splits-1 in order
// (matched_splitkv.py:121-126).  `row` is the (b, h) row of partials
// [splits][D]; this thread owns elements dd .. dd+E-1.  Splits are loaded kBatch
// at a time as straight-line vector loads; the first batch is issued before
// `prepare()` (which computes the weights), so the partial loads overlap the
// LSE loads and reductions (a scheduling barrier keeps them issued first).
// weight(s0, j) returns w_{s0+j}; it must be 0 for splits <= s0+j < 128 and
// finite for every index.  Past the last split the loads return zero, so the
// padding steps are fma(w, 0, acc) with w >= 0 finite and leave acc unchanged
// (acc is never -0: it starts at +0 and a round-to-nearest sum is -0 only if
// both addends are), so the batch size does not change the result's bits.
// w_s of a row whose weights lane l holds as w0 = w_l and w1 = w_{l+64}
// (lse_weights).  For s >= 128 it returns w_{s-64}, a finite value that only
// multiplies the zero a load past the row returns.
__device__ __forceinline__ float wave_weight(float w0, float w1, int s) {
  const float src = s < 64 ? w0 : w1;
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, src), s & 63));
}

template <int E>
struct MergeBatch {
  static constexpr int value = E == 1 ? 64 : (E == 2 ? 48 : (E == 4 ? 40 : (E == 8 ? 16 : 8)));
};

template <int E, bool kCoherent, typename PrepareFn, typename WeightFn>
__device__ __forceinline__ void merge_splits(const float* __restrict__ row, int D, int dd,
                                             int splits, PrepareFn prepare, WeightFn weight,
                                             float (&acc)[E]) {
  constexpr int kBatch = MergeBatch<E>::value;
  // `row` must be wavefront-uniform: the resource lives in scalar registers.
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(row, splits * D * 4);
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float x[kBatch][E];
  auto load = [&](int s0) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      buffer_load_f32<E, kCoherent>(rsrc, ((s0 + j) * D + dd) * 4, x[j]);
  };
  auto accumulate = [&](int s0) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const float wj = weight(s0, j);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = fmaf(wj, x[j][e], acc[e]);
    }
  };
  load(0);
  __builtin_amdgcn_sched_barrier(0);
  prepare();
  accumulate(0);
  for (int s0 = kBatch; s0 < splits; s0 += kBatch) {
    load(s0);
    accumulate(s0);
  }
}

// ------------------------------------------------------- matched partition
//
// Tile geometry: TILE = 16384 / D tokens (64/128/256 for D = 256/128/64), the
// reference's tile_tokens (splitkv_plan.py:33), so a tile is always 32 KiB of K
// and 32 KiB of V and never crosses a 256-token page.  Wavefront w owns tokens
// [w*TILE/4, (w+1)*TILE/4) of every tile, in groups of 16, for both products.
//
// QK^T on v_mfma_f32_16x16x32_bf16: A = K rows (lane L -> token L%16, d = 32c +
// 8*(L/16) .. +8, loaded straight into registers), B = Q of the GQA group
// (lane -> head L%16), so lane L holds S[token 4*(L/16)+r][head L%16],
// r = 0..3.  Padded heads (>= G) have zero Q and zero probabilities.
//
// PV on MFMA, with the bf16 probabilities as the A operand taken directly from
// the QK result registers: lane L holds P[head L%16][tokens 4*(L/16) + r] of
// each 16-token group, the A layout of v_mfma_f32_16x16x16_bf16 for one group
// and, for two groups g, g+1 side by side, of v_mfma_f32_16x16x32_bf16
// (k = 8*(L/16) + e <-> token 16g + 4*(L/16) + e for e < 4, 16(g+1) +
// 4*(L/16) + e-4 above).  The B operand needs V columns (4 consecutive tokens
// of one d per lane).  V rows therefore go to LDS by buffer_load ... lds (no
// registers; lane l of a copy fills bytes 16l .. 16l+15 of its 1 KiB, and
// reads past the buffer write zeros), each row padded by 16 bytes so that
// the transposed reads hit distinct banks, and are read with
// ds_read_b64_tr_b16: in each 16-lane group, when source lane 4c + b
// addresses row c, columns 4b .. 4b+3 of a 4 x 16 block, lane n receives
// column n of the block (rows 0..3).  Output lane L holds O[head 4*(L/16) + r]
// [d = 16j + L%16] of column block j.
template <int D, int GP>
struct Matched {
  static constexpr int kTile = 16384 / D;
  static constexpr int kTW = kTile / 4;                      // tokens per wavefront
  static constexpr int kNG = kTW / 16;                       // 16-token groups per wavefront
  static constexpr int kCH = D / 32;                         // 32-wide k-chunks of QK
  static constexpr int kNB = D / 16;                         // 16-column blocks of PV
  static constexpr int kPieces = D / 8 + 1;                  // 16-byte pieces per LDS row
  static constexpr int kPitch = 16 * kPieces;                // bytes per V row in LDS
  static constexpr int kDma = (kTW * kPitch + 1023) / 1024;  // 1 KiB copies per wavefront
  static constexpr int kSlot = 1024 * kDma;                  // LDS bytes of a wavefront's rows
  static constexpr int kOut = GP * D;                        // outputs of one GQA group
  static constexpr int kE = kOut >= kThreads ? kOut / kThreads : 1;  // per thread
  static_assert(kNG >= 1 && kCH >= 1 && 2 * kOut * 4 <= 4 * kSlot, "geometry");
};

template <int D, int GP>
struct KTile {
  u32x4_t k[Matched<D, GP>::kNG][Matched<D, GP>::kCH];
};

typedef short short4_t __attribute__((ext_vector_type(4)));

// 16 bytes at byte offset `off` of a buffer (zero past its end).
__device__ __forceinline__ u32x4_t buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int off) {
  const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
  return t;
}

// Four bf16 of one column, transposed out of LDS (see above).  `p` points
// into a __shared__ array; the LDS address-space casts live in these helpers
// so that kernel bodies only handle ordinary pointers.
__device__ __forceinline__ short4_t lds_read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4_t*)(const_cast<char*>(p)));
}

// Copies 16 bytes at byte offset `off` of a buffer into LDS: lane l of the
// wavefront writes bytes [dst + 16l, dst + 16l + 16); `dst` is wavefront-uniform.
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t rsrc, char* dst, int off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)dst, 16,
                                           off, 0, 0, 0);
}

// Workgroup barrier for LDS data written with ds_write only.  __syncthreads()
// also waits for every outstanding vector-memory operation, including the
// LDS copies of the next tile that are meant to stay in flight; this waits
// for the LDS instructions only.  The memory clobber keeps the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait states between the last MFMA writing `x` and the first vector-ALU read
// of it.  The hardware does not interlock this dependency, and this compiler
// emitted none when a branch separated the MFMA from the read: rows 8-15 of
// the 16x16 result were then read before the MFMA had written them.  24 wait
// states cover the 8-pass MFMAs used here; the empty statements keep every
// element's reads after them.
template <int N>
__device__ __forceinline__ void mfma_result_barrier(floatx4_t (&x)[N]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(x[N - 1]));
#pragma unroll
  for (int i = 0; i < N - 1; ++i) asm volatile("" : "+v"(x[i]));
}

// bf16 bits of (a, b), round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(floatx2_t{a, b}, bf16x2_t));
}

// Block-table window of one sequence: lane `lane` holds in e[r] the entry of
// page first + 64 r + lane (r < kRegs), loaded unconditionally through a
// buffer over the row's `width` entries (zero past the row), so the loads
// issue at kernel entry in the same round trip as the sequence length.
// page(t0) of a tile inside the window is a readlane; past the window it is
// a load of the entry (zero past the row, so a length beyond width * 256 reads
// page 0 instead of memory outside the table).
template <int kRegs>
struct PageWindow {
  const int32_t* row;
  int width, first;
  int32_t e[kRegs];

  __device__ __forceinline__ void load(const int32_t* __restrict__ trow, int width_, int first_,
                                       int lane) {
    row = trow;
    width = width_;
    first = first_;
    const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(trow, width_ * 4);
#pragma unroll
    for (int r = 0; r < kRegs; ++r)
      e[r] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, (first_ + 64 * r + lane) * 4, 0, 0);
  }

  // Waits for the window loads once, here, so that no later wait counts them
  // (the compiler cannot tell on every path that they have completed).
  __device__ __forceinline__ void settle() {
#pragma unroll
    for (int r = 0; r < kRegs; ++r) asm volatile("" : "+v"(e[r]));
  }

  // Page of logical token t0 (t0 >= first * 256, wavefront-uniform).
  __device__ __forceinline__ int page(int t0) const {
    const int idx = (t0 >> 8) - first;
    if (idx < 64 * kRegs) {
      int pg = __builtin_amdgcn_readlane(e[0], idx & 63);
#pragma unroll
      for (int r = 1; r < kRegs; ++r) {
        const int x = __builtin_amdgcn_readlane(e[r], idx & 63);
        pg = (idx >> 6) == r ? x : pg;
      }
      return pg;
    }
    return (t0 >> 8) < width ? row[t0 >> 8] : 0;
  }
};

// The K and V rows of one tile as buffers that end after row nvalid - 1, so
// rows past the sequence end read as zero without being fetched (NaN-poisoned
// slots and dead pages are never touched) and every load is unconditional.
// Byte sizes fit 32 bits: nvalid <= 256 and Hkv*D*512 < 2^31 (launcher check).
struct TileBuffers {
  __amdgpu_buffer_rsrc_t k, v;
};

__device__ __forceinline__ TileBuffers tile_buffers(const uint16_t* __restrict__ k,
                                                    const uint16_t* __restrict__ v, int page,
                                                    int t0, int end, int64_t RS, int kh, int D) {
  const int64_t base = (int64_t(page) * 256 + (t0 & 255)) * RS + int64_t(kh) * D;
  const int bytes = (end - t0 < 256 ? end - t0 : 256) * int(RS) * 2;
  return {buffer_rsrc(k + base, bytes), buffer_rsrc(v + base, bytes)};
}

template <int D, int GP>
struct MatchedShared {
  float wmax[2][4][16];  // per-tile maxima, double-buffered by tile parity
  float lsum[4][16];
  float mfin[16];
  int last;
};

// kFused = false: the partition alone (pd_partition).
// kFused = true: after writing its partial, each workgroup releases it at
// device scope and increments counters[b, kh]; the workgroup that completes
// the count acquires, merges all splits of its GQA group into `out` with the
// same arithmetic as lse_merge_kernel, and resets the counter to 0, so the
// counters are zero again when the kernel ends (graph replays need no reset).
template <int D, int GP, bool kFused>
__global__ void __launch_bounds__(kThreads, 2)
matched_partition_kernel(const uint16_t* __restrict__ q, int64_t qsb, int64_t qsh,
                         const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                         const int32_t* __restrict__ table, int64_t tsb, int width,
                         const int32_t* __restrict__ lengths, float* __restrict__ partials,
                         float* __restrict__ lse_out, int* __restrict__ counters,
                         uint16_t* __restrict__ out, int Hq, int Hkv, int G, int splits, int T,
                         float scale, float c) {
  using C = Matched<D, GP>;
  constexpr int TILE = C::kTile;
  __shared__ MatchedShared<D, GP> sm;
  // V rows of the tile being computed and of the one being loaded; two arrays
  // (not one) so that the compiler's wait before reading one slot does not
  // count the copies still in flight into the other.
  __shared__ __attribute__((aligned(16))) char vs0[4 * C::kSlot];
  __shared__ __attribute__((aligned(16))) char vs1[4 * C::kSlot];

  const int p = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qh = lane & 15, qg = lane >> 4;
  const int start = p * T;
  // The partition's table entries do not depend on the length: fetch them
  // together with it, so the first KV loads wait for one round trip.
  PageWindow<2> pw;
  pw.load(table + int64_t(b) * tsb, width, start >> 8, lane);
  const int length = lengths[b];
  const int end = min(start + T, length);
  const int count = end > start ? (end - start + TILE - 1) / TILE : 0;
  const int64_t RS = int64_t(Hkv) * D;

  // MFMA B operand of QK: the GQA group's query rows.
  bf16x8_t qf[C::kCH];
  {
    const bool live = qh < G;
    const uint16_t* qrow =
        q + int64_t(b) * qsb + int64_t(kh * G + (live ? qh : 0)) * qsh + 8 * qg;
#pragma unroll
    for (int ch = 0; ch < C::kCH; ++ch)
      qf[ch] = __builtin_bit_cast(bf16x8_t, live ? load16(qrow + 32 * ch) : u32x4_t{0, 0, 0, 0});
  }

  // Tile-relative byte offsets: K pieces of this lane, and the source of
  // each 16-byte LDS piece this lane fills (row, piece) = (slot / kPieces,
  // slot % kPieces); the padding piece and rows past the wavefront's share
  // read past the buffer, i.e. zeros.
  const int koff = ((w * C::kTW + qh) * int(RS) + 8 * qg) * 2;
  int voff[C::kDma];
#pragma unroll
  for (int i = 0; i < C::kDma; ++i) {
    const int slot = 64 * i + lane;
    const int row = slot / C::kPieces, piece = slot % C::kPieces;
    voff[i] = row < C::kTW && piece < D / 8 ? ((w * C::kTW + row) * int(RS) + 8 * piece) * 2
                                            : 0x7ffffff0;
  }
  // This lane's transposed-read address within its wavefront's LDS rows.
  const int trb = w * C::kSlot + (4 * qg + ((lane & 15) >> 2)) * C::kPitch + 8 * (lane & 3);

  floatx4_t acc[C::kNB];   // O[head 4*qg + r][16j + qh]
#pragma unroll
  for (int j = 0; j < C::kNB; ++j) acc[j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  float m4[4];             // running max of heads 4*qg + r
#pragma unroll
  for (int r = 0; r < 4; ++r) m4[r] = -INFINITY;
  float m_own = -INFINITY;  // running max of head qh
  float l_own = 0.f;        // this lane's share of head qh's denominator

  // Issues the loads of tile ti (ti < 0: an empty load, nothing fetched).
  auto issue = [&](KTile<D, GP>& R, char* slot, int ti) __attribute__((always_inline)) {
    const int t0 = start + (ti > 0 ? ti : 0) * TILE;
    const TileBuffers buf = tile_buffers(k, v, pw.page(t0), t0, ti >= 0 ? end : t0, RS, kh, D);
#pragma unroll
    for (int g = 0; g < C::kNG; ++g)
#pragma unroll
      for (int ch = 0; ch < C::kCH; ++ch)
        R.k[g][ch] = buffer_load16(buf.k, koff + g * 16 * int(RS) * 2 + 64 * ch);
#pragma unroll
    for (int i = 0; i < C::kDma; ++i)
      lds_copy16(buf.v, slot + w * C::kSlot + 1024 * i, voff[i]);
  };

  auto process = [&](const KTile<D, GP>& R, const char* slot, int ti)
                     __attribute__((always_inline)) {
    const int nvalid = end - (start + ti * TILE);
    // ---- scores
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
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float (*wm)[16] = sm.wmax[ti & 1];
    if (lane < 16) wm[w][lane] = mx;
    lds_barrier();
    // ---- running maxima (reference order: m' = max(m, rowmax s))
    float alpha[4];
    bool moved = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * qg + r;
      const float tm = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
      const float mn = fmaxf(m4[r], tm);
      moved |= mn != m4[r];
      alpha[r] = exp2_fast((m4[r] - mn) * c);
      m4[r] = mn;
    }
    const float tm = fmaxf(fmaxf(wm[0][qh], wm[1][qh]), fmaxf(wm[2][qh], wm[3][qh]));
    const float mn = fmaxf(m_own, tm);
    const float a_own = exp2_fast((m_own - mn) * c);
    m_own = mn;
    const float neg_mc = -(mn * c);
    float psum = 0.f;
    uint32_t pb[C::kNG][2];  // bf16 probabilities, the PV A operand
#pragma unroll
    for (int g = 0; g < C::kNG; ++g) {
      float pr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = exp2_fast(fmaf(s[g][r], c, neg_mc));
        psum += pr[r];
      }
      pb[g][0] = qh < G ? pack_bf16(pr[0], pr[1]) : 0u;
      pb[g][1] = qh < G ? pack_bf16(pr[2], pr[3]) : 0u;
    }
    l_own = l_own * a_own + psum;
    // ---- PV (rescale only when a running maximum moved; alpha = 1 otherwise)
    if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
      for (int j = 0; j < C::kNB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] *= alpha[r];
    }
    const char* base = slot + trb;
    if constexpr (C::kNG == 1) {
      const short4_t a = __builtin_bit_cast(short4_t, u32x2_t{pb[0][0], pb[0][1]});
#pragma unroll
      for (int j = 0; j < C::kNB; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, lds_read_tr(base + 32 * j), acc[j],
                                                           0, 0, 0);
    } else {
#pragma unroll
      for (int g = 0; g < C::kNG; g += 2) {
        const bf16x8_t a =
            __builtin_bit_cast(bf16x8_t, u32x4_t{pb[g][0], pb[g][1], pb[g + 1][0], pb[g + 1][1]});
#pragma unroll
        for (int j = 0; j < C::kNB; ++j) {
          const short4_t lo = lds_read_tr(base + 16 * g * C::kPitch + 32 * j);
          const short4_t hi = lds_read_tr(base + 16 * (g + 1) * C::kPitch + 32 * j);
          const bf16x8_t bv = __builtin_bit_cast(
              bf16x8_t, u32x4_t{__builtin_bit_cast(u32x2_t, lo)[0], __builtin_bit_cast(u32x2_t, lo)[1],
                                __builtin_bit_cast(u32x2_t, hi)[0], __builtin_bit_cast(u32x2_t, hi)[1]});
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bv, acc[j], 0, 0, 0);
        }
      }
    }
  };

  // Reverse tile walk (matched_splitkv.py:71): last tile first.  Two register
  // sets and two LDS slots alternate: the loads of the next tile are issued
  // before the current one is computed.  The load after the last tile is an
  // empty one (a buffer of 0 bytes, nothing fetched), so every iteration
  // issues the same loads.
  pw.settle();
  if (count > 0) {
    KTile<D, GP> A, B;
    int ti = count - 1;
    issue(A, vs0, ti);
    while (true) {
      issue(B, vs1, ti - 1);
      process(A, vs0, ti);
      if (--ti < 0) break;
      issue(A, vs0, ti - 1);
      process(B, vs1, ti);
      if (--ti < 0) break;
    }
  }

  // ---- epilogue: combine the 4 waves' accumulators and denominators
  float l = l_own;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (lane < 16) sm.lsum[w][lane] = l;
  if (tid < 16) sm.mfin[tid] = m_own;
  __syncthreads();  // every wavefront is done with its V rows (aliased by red)
  // O of wavefront w for the group's heads: waves 0, 1 in vs0, waves 2, 3 in vs1.
  auto red = [&](int wave) __attribute__((always_inline)) {
    return reinterpret_cast<float*>(wave < 2 ? vs0 : vs1) + (wave & 1) * C::kOut;
  };
  {
    float* mine = red(w);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * qg + r;
      if (h < GP)
#pragma unroll
        for (int j = 0; j < C::kNB; ++j) mine[h * D + 16 * j + qh] = acc[j][r];
    }
  }
  lds_barrier();

  const int idx0 = tid * C::kE;
  const int h = idx0 / D, dd = idx0 % D;  // kE divides D, so one head per thread
  if (idx0 < C::kOut && h < G) {
    const float den = (sm.lsum[0][h] + sm.lsum[1][h]) + (sm.lsum[2][h] + sm.lsum[3][h]);
    const float safe = den > 0.f ? den : 1.f;
    const float inv = rcp_fast(safe);
    const int64_t orow = (int64_t(b) * Hq + kh * G + h) * splits + p;
    float* dst = partials + orow * D + dd;
    const float lv = den > 0.f ? fmaf(sm.mfin[h], scale, ln_fast(safe)) : -INFINITY;
    float val[C::kE];
#pragma unroll
    for (int e = 0; e < C::kE; ++e) {
      const int i = idx0 + e;
      val[e] = ((red(0)[i] + red(1)[i]) + (red(2)[i] + red(3)[i])) * inv;
    }
    if constexpr (kFused) {
      // Device-scope stores (global_store sc1): written through to the
      // coherence point, so another XCD can read them without any L2 flush.
#pragma unroll
      for (int e = 0; e < C::kE; ++e)
        __hip_atomic_store(dst + e, val[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (dd == 0) __hip_atomic_store(lse_out + orow, lv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
#pragma unroll
      for (int e = 0; e < C::kE; ++e) dst[e] = val[e];
      if (dd == 0) lse_out[orow] = lv;
    }
  }

  if constexpr (kFused) {
    // Split-completion count.  Every partial and LSE value exchanged between
    // workgroups is written and read with device-scope (sc1) accesses.  The
    // barrier waits until this workgroup's stores have completed before thread
    // 0 increments the counter, and the last workgroup issues its loads only
    // after its increment returned splits - 1, i.e. after every other
    // workgroup's stores completed.  No cache-wide writeback or invalidate is
    // needed, so the KV tiles other calls keep in L2 stay resident.
    int* counter = counters + int64_t(b) * Hkv + kh;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (tid == 0)
      sm.last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                splits - 1;
    __syncthreads();
    if (!sm.last) return;
    // Wavefront w merges query heads w, w + 4, ... of the group; lane owns
    // D/64 consecutive columns, as in lse_merge_kernel's wavefronts.
    const int64_t row0 = int64_t(b) * Hq + kh * G;  // first query head of the group
    constexpr int kV = D / 64;
    for (int hh = __builtin_amdgcn_readfirstlane(w); hh < G; hh += 4) {
      float w0 = 0.f, w1 = 0.f, acc[kV];
      merge_splits<kV, true>(
          partials + (row0 + hh) * splits * D, D, lane * kV, splits,
          [&] { lse_weights<true>(lse_out + (row0 + hh) * splits, splits, lane, w0, w1); },
          [&](int s0, int j) { return wave_weight(w0, w1, s0 + j); }, acc);
      uint16_t* dst = out + (row0 + hh) * D + lane * kV;
#pragma unroll
      for (int e = 0; e < kV; ++e) dst[e] = uint16_t(bf16_bits(acc[e]));
    }
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------- LSE merge
// One workgroup of D threads per (b, h) row, one output element per thread.
// Every wavefront computes the row's weights itself (the same arithmetic, so
// the same bits) and broadcasts them with readlane: no LDS, no barrier.
template <int D>
__global__ void __launch_bounds__(D)
lse_merge_kernel(const float* __restrict__ partials, const float* __restrict__ lse,
                 uint16_t* __restrict__ out, int splits) {
  const int64_t row = blockIdx.x;
  const int dd = threadIdx.x;
  const int lane = dd & 63;
  float w0 = 0.f, w1 = 0.f, acc[1];
  merge_splits<1, false>(
      partials + row * splits * D, D, dd, splits,
      [&] { lse_weights<false>(lse + row * splits, splits, lane, w0, w1); },
      [&](int s0, int j) { return wave_weight(w0, w1, s0 + j); }, acc);
  out[row * D + dd] = uint16_t(bf16_bits(acc[0]));
}

// ------------------------------------------------- base / fixed-split kernel
//
// One 256-thread workgroup per (b, h[, partition]).  Each row of K/V is read
// by D/8 lanes (16 bytes each); the 256/(D/8) row groups walk 16384/D-token
// tiles (one page each), every row group keeping its own (m, l, acc) state
// with fp32 p, merged across row groups and waves at the end.  With fp32
// probabilities the result does not depend on the tile schedule beyond
// float32 rounding.
template <int D>
struct Online {
  static constexpr int kLPR = D / 8;
  static constexpr int kRG = kThreads / kLPR;
  static constexpr int kTile = 8 * kRG;  // 16384 / D
};

template <int D, bool kSplit>
__global__ void __launch_bounds__(kThreads)
online_decode_kernel(const uint16_t* __restrict__ q, int64_t qsb, int64_t qsh,
                     const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                     const int32_t* __restrict__ table, int64_t tsb, int width,
                     const int32_t* __restrict__ lengths, uint16_t* __restrict__ out,
                     float* __restrict__ maxima, float* __restrict__ denoms,
                     float* __restrict__ accums, int Hq, int Hkv, int G, int parts,
                     int part_size, float scale) {
  using C = Online<D>;
  constexpr int TILE = C::kTile;
  constexpr int LPR = C::kLPR;
  __shared__ float wm[4], wl[4];
  __shared__ float wacc[4][D];

  const int part = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rg = tid / LPR, d0 = (tid % LPR) * 8;
  const int kh = h / G;
  const int start = kSplit ? part * part_size : 0;
  PageWindow<1> pw;  // fetched with the length, as in the matched partition
  pw.load(table + int64_t(b) * tsb, width, start >> 8, lane);
  const int length = lengths[b];
  const int end = kSplit ? min(start + part_size, length) : length;
  const int64_t RS = int64_t(Hkv) * D;

  const u32x4_t qv = load16(q + int64_t(b) * qsb + int64_t(h) * qsh + d0);

  float m = -INFINITY, l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;

  pw.settle();
  for (int t0 = start; t0 < end; t0 += TILE) {
    const TileBuffers buf = tile_buffers(k, v, pw.page(t0), t0, end, RS, kh, D);
    const int nvalid = end - t0;
    u32x4_t kr[8], vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int off = ((rg + i * C::kRG) * int(RS) + d0) * 2;
      kr[i] = buffer_load16(buf.k, off);
      vr[i] = buffer_load16(buf.v, off);
    }
    __builtin_amdgcn_sched_barrier(0);  // all 16 loads in flight before the first use
    float s[8];
    float smax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) x = dot2(kr[i][e], qv[e], x);
#pragma unroll
      for (int msk = 1; msk < LPR; msk <<= 1) x += __shfl_xor(x, msk);
      x *= scale;
      s[i] = rg + i * C::kRG < nvalid ? x : -INFINITY;
      smax = fmaxf(smax, s[i]);
    }
    const float mn = fmaxf(m, smax);
    // A row group with no valid row so far keeps m = -inf; subtract 0 instead
    // of -inf so that exp(-inf - -inf) never turns the empty state into NaN.
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float alpha = exp_fast(m - mref);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pr = exp_fast(s[i] - mref);
      l += pr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] = fmaf(pr, bf16_lo(vr[i][e]), acc[2 * e]);
        acc[2 * e + 1] = fmaf(pr, bf16_hi(vr[i][e]), acc[2 * e + 1]);
      }
    }
    m = mn;
  }

  // Merge row groups inside the wave (lanes sharing d0), then across waves.
#pragma unroll
  for (int msk = LPR; msk < 64; msk <<= 1) {
    const float mo = __shfl_xor(m, msk);
    const float lo = __shfl_xor(l, msk);
    const float mn = fmaxf(m, mo);
    const float fa = m == -INFINITY ? 0.f : exp_fast(m - mn);
    const float fb = mo == -INFINITY ? 0.f : exp_fast(mo - mn);
    l = l * fa + lo * fb;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = acc[e] * fa + __shfl_xor(acc[e], msk) * fb;
    m = mn;
  }
  if (lane == 0) {
    wm[w] = m;
    wl[w] = l;
  }
  if (lane < LPR)
#pragma unroll
    for (int e = 0; e < 8; ++e) wacc[w][d0 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    float mx = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    float f[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) f[x] = wm[x] == -INFINITY ? 0.f : exp_fast(wm[x] - mx);
    const float tot = (wl[0] * f[0] + wl[1] * f[1]) + (wl[2] * f[2] + wl[3] * f[3]);
    const float num = (wacc[0][tid] * f[0] + wacc[1][tid] * f[1]) +
                      (wacc[2][tid] * f[2] + wacc[3][tid] * f[3]);
    if constexpr (kSplit) {
      const int64_t idx = (int64_t(b) * Hq + h) * parts + part;
      accums[idx * D + tid] = num;
      if (tid == 0) {
        maxima[idx] = mx;
        denoms[idx] = tot;
      }
    } else {
      out[(int64_t(b) * Hq + h) * D + tid] = uint16_t(bf16_bits(num / (tot > 0.f ? tot : 1.f)));
    }
  }
}

// ------------------------------------------------------------ m/l/acc merge
template <int VEC>
__global__ void __launch_bounds__(64)
ml_merge_kernel(const float* __restrict__ maxima, const float* __restrict__ denoms,
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
  if (int64_t(num_kv_heads) * head_dim * 512 >= (int64_t(1) << 31))
    return pd::fail(PD_EINVAL, "a 256-slot page of one KV tensor must stay below 2 GiB");
  if (width < 1 || width >= (1 << 22))
    return pd::fail(PD_EINVAL, "table width must be in [1, 2^22)");
  return PD_OK;
}

struct PartitionArgs {
  const uint16_t* q;
  int64_t qsb, qsh;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* table;
  int64_t tsb;
  int width;
  const int32_t* lengths;
  float* partials;
  float* lse;
  int* counters;
  uint16_t* out;
  int Hq, Hkv, G, splits, T;
  float scale, c;
};

template <int D, bool kFused>
void launch_partition_d(int gp, dim3 grid, hipStream_t stream, const PartitionArgs& a) {
#define PD_LAUNCH_GP(GPV)                                                                     \
  hipLaunchKernelGGL((matched_partition_kernel<D, GPV, kFused>), grid, dim3(kThreads), 0,     \
                     stream, a.q, a.qsb, a.qsh, a.k, a.v, a.table, a.tsb, a.width,          \
                     a.lengths, a.partials, a.lse, a.counters, a.out, a.Hq, a.Hkv, a.G,       \
                     a.splits, a.T, a.scale, a.c)
  switch (gp) {
    case 1: PD_LAUNCH_GP(1); break;
    case 2: PD_LAUNCH_GP(2); break;
    case 4: PD_LAUNCH_GP(4); break;
    case 8: PD_LAUNCH_GP(8); break;
    default: PD_LAUNCH_GP(16); break;
  }
#undef PD_LAUNCH_GP
}

int padded_group(int g) {
  int gp = 1;
  while (gp < g) gp <<= 1;
  return gp;
}

// Validation and dispatch shared by pd_partition (fused = false) and
// pd_matched_decode (fused = true).
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
  PartitionArgs a{static_cast<const uint16_t*>(q), qsb, qsh, static_cast<const uint16_t*>(k),
                  static_cast<const uint16_t*>(v), table, tsb, width, lengths, partials, lse,
                  counters, static_cast<uint16_t*>(out), num_heads, num_kv_heads, G, splits,
                  tokens_per_split, float(scale),
                  float(scale * 1.4426950408889634)};  // SCALE_LOG2 (matched_splitkv.py:363)
  const dim3 grid(splits, num_kv_heads, batch);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int gp = padded_group(G);
  switch (head_dim * 2 + (fused ? 1 : 0)) {
    case 128: launch_partition_d<64, false>(gp, grid, st, a); break;
    case 129: launch_partition_d<64, true>(gp, grid, st, a); break;
    case 256: launch_partition_d<128, false>(gp, grid, st, a); break;
    case 257: launch_partition_d<128, true>(gp, grid, st, a); break;
    case 512: launch_partition_d<256, false>(gp, grid, st, a); break;
    default: launch_partition_d<256, true>(gp, grid, st, a); break;
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

extern "C" int pd_matched_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                 const void* k, const void* v, const int32_t* table,
                                 int64_t table_stride_b, int32_t table_width,
                                 const int32_t* lengths, float* partials, float* lse,
                                 int32_t* counters, void* out,
                                 int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t splits, int32_t tokens_per_split,
                                 int32_t tile_tokens, double scale, pd_stream_t stream) {
  return partition_entry("pd_matched_decode", true, q, q_stride_b, q_stride_h, k, v, table,
                         table_stride_b, table_width, lengths, partials, lse, counters, out,
                         batch,
                         num_heads, num_kv_heads, head_dim, splits, tokens_per_split,
                         tile_tokens, scale, stream);
}

extern "C" int pd_lse_merge(const float* partials, const float* lse, void* out, int32_t batch,
                            int32_t num_heads, int32_t head_dim, int32_t splits,
                            int32_t lse_lanes, pd_stream_t stream) {
  pd::clear_error();
  if (batch <= 0 || num_heads <= 0) return pd::fail(PD_EINVAL, "batch and heads must be positive");
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (splits < 1 || splits > 128) return pd::fail(PD_EINVAL, "splits must be in [1,128]");
  if (lse_lanes < 1 || (lse_lanes & (lse_lanes - 1)))
    return pd::fail(PD_EINVAL, "lse_lanes must be a power of two");
  if (!partials || !lse || !out) return pd::fail(PD_EINVAL, "null tensor pointer");
  if (!aligned16(partials)) return pd::fail(PD_EINVAL, "partials must be 16-byte aligned");
  const int64_t rows = int64_t(batch) * num_heads;
  if (rows > 0x7fffffff) return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto* o = static_cast<uint16_t*>(out);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(lse_merge_kernel<64>, dim3(rows), dim3(64), 0, st, partials, lse, o, splits);
      break;
    case 128:
      hipLaunchKernelGGL(lse_merge_kernel<128>, dim3(rows), dim3(128), 0, st, partials, lse, o, splits);
      break;
    default:
      hipLaunchKernelGGL(lse_merge_kernel<256>, dim3(rows), dim3(256), 0, st, partials, lse, o, splits);
      break;
  }
  return launch_status("pd_lse_merge");
}

namespace {

template <bool kSplit>
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
  if (batch > 65535 || num_heads > 65535)
    return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  if (kSplit) {
    if (parts < 1) return pd::fail(PD_EINVAL, "partitions must be positive");
    if (part_size <= 0 || part_size % (16384 / head_dim))
      return pd::fail(PD_EINVAL, "partition_size must be a positive multiple of %d",
                      16384 / head_dim);
    if (int64_t(parts) * part_size >= (int64_t(1) << 31))
      return pd::fail(PD_EINVAL, "partitions * partition_size must stay below 2^31");
    if (!maxima || !denoms || !accums)
      return pd::fail(PD_EINVAL, "invalid or missing preallocated split-K workspace");
  } else if (!out) {
    return pd::fail(PD_EINVAL, "invalid output buffer");
  }
  const int G = num_heads / num_kv_heads;
  const dim3 grid(kSplit ? parts : 1, num_heads, batch);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const auto* qq = static_cast<const uint16_t*>(q);
  const auto* kk = static_cast<const uint16_t*>(k);
  const auto* vv = static_cast<const uint16_t*>(v);
  auto* o = static_cast<uint16_t*>(out);
  const float s32 = float(scale);
#define PD_LAUNCH_ONLINE(DV)                                                                  \
  hipLaunchKernelGGL((online_decode_kernel<DV, kSplit>), grid, dim3(kThreads), 0, st, qq, qsb, \
                     qsh, kk, vv, table, tsb, width, lengths, o, maxima, denoms, accums,      \
                     num_heads, num_kv_heads, G, parts, part_size, s32)
  switch (head_dim) {
    case 64: PD_LAUNCH_ONLINE(64); break;
    case 128: PD_LAUNCH_ONLINE(128); break;
    default: PD_LAUNCH_ONLINE(256); break;
  }
#undef PD_LAUNCH_ONLINE
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
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto* o = static_cast<uint16_t*>(out);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(ml_merge_kernel<1>, dim3(rows), dim3(64), 0, st, maxima, denoms, accums, o, partitions);
      break;
    case 128:
      hipLaunchKernelGGL(ml_merge_kernel<2>, dim3(rows), dim3(64), 0, st, maxima, denoms, accums, o, partitions);
      break;
    default:
      hipLaunchKernelGGL(ml_merge_kernel<4>, dim3(rows), dim3(64), 0, st, maxima, denoms, accums, o, partitions);
      break;
  }
  return launch_status("pd_ml_merge");
}

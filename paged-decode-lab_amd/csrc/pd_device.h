// Device-side building blocks shared by the paged decode kernels for MI355X
// (gfx950, CDNA4): numerics, buffer-resource loads, the LSE merge arithmetic,
// the matched-partition tile geometry, LDS copy/transposed-read helpers and
// the block-table window.  Included by the kernel translation units only.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace pdk {

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

// x of lane L ^ M, for M = 1, 2, 4, 8, 16 or 32, with VALU lane moves (no LDS
// round trip, unlike ds_bpermute).  Lane layouts checked on gfx950 with an
// in-bounds probe: DPP quad_perm [1,0,3,2] / [2,3,0,1] give L ^ 1 / L ^ 2;
// row_shl:n gives lane L + n of the same 16-lane row and row_shr:n lane L - n,
// so L ^ 4 and L ^ 8 select between the two by the lane bit; for
// v_permlane16_swap(x, x) the first result holds x[L ^ 16] in the odd 16-lane
// rows and the second in the even rows, and v_permlane32_swap likewise for
// the upper / lower 32 lanes.
template <int M>
__device__ __forceinline__ float xor_lanes(float x, int lane) {
  const int v = __float_as_int(x);
  if constexpr (M == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));
  } else if constexpr (M == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));
  } else if constexpr (M == 4 || M == 8) {
    const int up = __builtin_amdgcn_mov_dpp(v, 0x100 + M, 0xF, 0xF, false);  // row_shl:M
    const int dn = __builtin_amdgcn_mov_dpp(v, 0x110 + M, 0xF, 0xF, false);  // row_shr:M
    return __int_as_float((lane & M) ? dn : up);
  } else if constexpr (M == 16) {
    const auto a = __builtin_amdgcn_permlane16_swap(unsigned(v), unsigned(v), false, false);
    return __uint_as_float((lane & 16) ? a[0] : a[1]);
  } else {
    static_assert(M == 32, "xor distance");
    const auto a = __builtin_amdgcn_permlane32_swap(unsigned(v), unsigned(v), false, false);
    return __uint_as_float((lane & 32) ? a[0] : a[1]);
  }
}

// x of lane L ^ m for any m in [0, 64) (wavefront-uniform), one move per set bit.
__device__ __forceinline__ float xor_lanes_any(float x, int m, int lane) {
  if (m & 32) x = xor_lanes<32>(x, lane);
  if (m & 16) x = xor_lanes<16>(x, lane);
  if (m & 8) x = xor_lanes<8>(x, lane);
  if (m & 4) x = xor_lanes<4>(x, lane);
  if (m & 2) x = xor_lanes<2>(x, lane);
  if (m & 1) x = xor_lanes<1>(x, lane);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  const int lane = __lane_id();
  x = fmaxf(x, xor_lanes<32>(x, lane));
  x = fmaxf(x, xor_lanes<16>(x, lane));
  x = fmaxf(x, xor_lanes<8>(x, lane));
  x = fmaxf(x, xor_lanes<4>(x, lane));
  x = fmaxf(x, xor_lanes<2>(x, lane));
  return fmaxf(x, xor_lanes<1>(x, lane));
}

// Sum over the 64 lanes: an xor butterfly at distances 32, 16, ..., 1.  Each
// step adds the same two values in every lane of a pair (float addition
// commutes), so every lane ends with the same bits.
__device__ __forceinline__ float wave_sum(float x) {
  const int lane = __lane_id();
  x += xor_lanes<32>(x, lane);
  x += xor_lanes<16>(x, lane);
  x += xor_lanes<8>(x, lane);
  x += xor_lanes<4>(x, lane);
  x += xor_lanes<2>(x, lane);
  return x + xor_lanes<1>(x, lane);
}

// Reductions over the four 16-lane rows of a wavefront (lanes L, L^16, L^32,
// L^48) with v_permlane16_swap / v_permlane32_swap: each swap returns the
// pair {x[L], x[L^16]} (or {x[L], x[L^32]}) in some order, so a commutative
// op over the pair is the same for every lane.  Pure VALU, no LDS traffic.
// The sum adds x[L] + x[L^16] first, then the xor-32 partner, the same
// association as a butterfly over shuffles at distance 16 then 32.
__device__ __forceinline__ float max_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ u32x4_t load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// Buffer resource (V#) over `bytes` bytes at `base`; word 3 is the gfx9-family
// raw-buffer format.  Loads at or past `bytes` return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Cache-policy operand of the buffer builtins (bit 0 is sc0, bit 1 nt, bit 4
// sc1).  kCoherentAux (sc1): device-scope coherent accesses, written through to
// / re-read from the coherence point beyond the XCDs' L2s, so a line another
// XCD wrote is seen.
constexpr int kCoherentAux = 16;

// E consecutive floats at byte offset `off`, with cache policy kAux.
// The builtins' results are bit-cast as whole vectors to float vectors before
// any element is read: reading elements of their integer vector results
// directly made this compiler emit a single dword load for the whole vector.
template <int E, int kAux>
__device__ __forceinline__ void buffer_load_f32(__amdgpu_buffer_rsrc_t rsrc, int off,
                                                float (&x)[E]) {
  constexpr int aux = kAux;
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
// The plan's LSE lane count for a split count and head dim:
// min(next_pow2(splits), 32 if D % 128 == 0 else 16) (splitkv_plan.py:52-56).
__device__ __host__ __forceinline__ int plan_lse_lanes(int splits, int D) {
  int lanes = 1;
  while (lanes < splits) lanes <<= 1;
  const int cap = D % 128 == 0 ? 32 : 16;
  return lanes < cap ? lanes : cap;
}

// Merge weights of one (b, h) row, computed by one full wavefront: lane owns
// splits `lane` and `lane + 64` (splits <= 128).  M = max lse (-inf -> 0),
// S = sum exp(lse - M), L = ln S + M (+inf when S == 0), w_p = exp(lse_p - L)
// (matched_splitkv.py:107-120; an all-empty row gets w = 0 everywhere).  The
// two loads are unconditional buffer loads (zero past the row, replaced by
// -inf), so they issue without a branch and queue behind earlier loads.
// S is summed in the reference's float32 order for `lanes` (a power of two,
// 1..64): lane j < lanes adds e_j, e_{j+lanes}, e_{j+2 lanes}, ... in that
// order (:114-118), then a halving tree over the lanes adds lane j + half to
// lane j (:119), here an xor butterfly (float addition commutes exactly).
// Terms past the last split are exact zeros, so they are not added.
// The two LSE loads of lse_weights (a row of `bytes` bytes; zero past it), so
// that a caller can issue several rows' loads before any is needed.
template <int kAux>
__device__ __forceinline__ void lse_load(const float* __restrict__ lrow, int bytes, int lane,
                                         float& a, float& c) {
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(lrow, bytes);
  float x[1], y[1];
  buffer_load_f32<1, kAux>(rsrc, lane * 4, x);
  buffer_load_f32<1, kAux>(rsrc, (lane + 64) * 4, y);
  a = x[0];
  c = y[0];
}

// lse_weights on the values lse_load returned for the row.
// Lane j < lanes needs e_{j + t lanes} for t = 1, 2, ...: split j + t lanes is
// element j + (t lanes & 63) of e0 (t lanes < 64) or e1, and since lanes is a
// power of two and j < lanes, j + (t lanes & 63) = j ^ (t lanes & 63), so
// every term is an xor move.  The plan's lane counts (capped at 32 for D 128
// and 256, 16 for D 64) take an unrolled path; any other power of two a caller
// passes takes the general loop.
__device__ __forceinline__ void lse_weights_of(float a, float c, int splits, int lanes, int lane,
                                               float& w0, float& w1) {
  const float v0 = lane < splits ? a : -INFINITY;
  const float v1 = lane + 64 < splits ? c : -INFINITY;
  float mx = wave_max(fmaxf(v0, v1));
  if (mx == -INFINITY) mx = 0.f;
  const float e0 = exp_fast(v0 - mx), e1 = exp_fast(v1 - mx);
  float s = e0;
  const int terms = (splits + lanes - 1) / lanes;
  if (terms > 1) {
    // Terms past the last split are exact zeros and are not added.
    const float e0x32 = xor_lanes<32>(e0, lane), e1x32 = xor_lanes<32>(e1, lane);
    if (lanes == 32) {
      s += e0x32;                        // t = 1: splits j + 32
      if (terms > 2) s += e1;            // t = 2: j + 64
      if (terms > 3) s += e1x32;         // t = 3: j + 96
    } else if (lanes != 16) {
      for (int t = 1; t < terms; ++t) {
        const int off = t * lanes;
        s += xor_lanes_any(off < 64 ? e0 : e1, off & 63, lane);
      }
    } else {
      const float e0x16 = xor_lanes<16>(e0, lane), e1x16 = xor_lanes<16>(e1, lane);
      const float e0x48 = xor_lanes<16>(e0x32, lane), e1x48 = xor_lanes<16>(e1x32, lane);
      s += e0x16;                        // j + 16
      if (terms > 2) s += e0x32;         // j + 32
      if (terms > 3) s += e0x48;         // j + 48
      if (terms > 4) s += e1;            // j + 64
      if (terms > 5) s += e1x16;         // j + 80
      if (terms > 6) s += e1x32;         // j + 96
      if (terms > 7) s += e1x48;         // j + 112
    }
  }
  // Halving tree: lane j adds lane j ^ m for m = lanes / 2, ..., 1.
  if (lanes > 32) s += xor_lanes<32>(s, lane);
  if (lanes > 16) s += xor_lanes<16>(s, lane);
  if (lanes > 8) s += xor_lanes<8>(s, lane);
  if (lanes > 4) s += xor_lanes<4>(s, lane);
  if (lanes > 2) s += xor_lanes<2>(s, lane);
  if (lanes > 1) s += xor_lanes<1>(s, lane);
  const float total = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), 0));
  const float logsum = total > 0.f ? ln_fast(total) + mx : INFINITY;
  w0 = exp_fast(v0 - logsum);
  w1 = exp_fast(v1 - logsum);
}

template <int kAux>
__device__ __forceinline__ void lse_weights(const float* __restrict__ lrow, int splits, int lanes,
                                            int lane, float& w0, float& w1) {
  float a, c;
  lse_load<kAux>(lrow, splits * 4, lane, a, c);
  lse_weights_of(a, c, splits, lanes, lane, w0, w1);
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

template <int E, int kAux, int kBatch = MergeBatch<E>::value, typename PrepareFn,
          typename WeightFn>
__device__ __forceinline__ void merge_splits(const float* __restrict__ row, int D, int dd,
                                             int splits, PrepareFn prepare, WeightFn weight,
                                             float (&acc)[E]) {
  // `row` must be wavefront-uniform: the resource lives in scalar registers.
  const __amdgpu_buffer_rsrc_t rsrc = buffer_rsrc(row, splits * D * 4);
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float x[kBatch][E];
  auto load = [&](int s0) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      buffer_load_f32<E, kAux>(rsrc, ((s0 + j) * D + dd) * 4, x[j]);
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

// ------------------------------------------------ (m, l, acc) online merge
// The merge of the fixed-split protocol's partition states, in the order the
// fixed-split walk completes them: p = P - 1 down to 0.  A partition with
// m_p = -inf holds no token and is skipped.  For the others, with M the
// maximum of the partitions merged so far (-inf before the first):
//   M' = max(M, m_p), a = exp(M - M'), b = exp(m_p - M'),
//   acc = fma(acc_p, b, acc * a), total = fma(l_p, b, total * a), M = M',
// and the output is acc * (1 / (total > 0 ? total : 1)).  This is the
// reference's merge (kernels.py:83-100: maximum first, then the factors
// exp(m_p - M)) computed as a running maximum, with its own float32 rounding.
// ml_online_merge_kernel and the walk's in-kernel merge (cols_loader_kernel)
// both use ml_step in that order, so the two give the same bits.
struct MlStep {
  float a, b;  // factor of the running state and of the partition
  bool live;   // m_p > -inf
};

__device__ __forceinline__ MlStep ml_step(float m_p, float& M) {
  // Without a branch: both exponentials are computed and selected away for an
  // empty partition (where M - mn may be -inf - (-inf)).
  const bool live = m_p != -INFINITY;
  const float mn = fmaxf(M, m_p);
  const float ea = exp_fast(M - mn), eb = exp_fast(m_p - mn);
  const MlStep st{live ? ea : 1.f, live ? eb : 0.f, live};
  M = live ? mn : M;
  return st;
}



// x of lane L + k, or -inf past lane 63 (k > 0, wavefront-uniform).  The
// lane move runs in every lane: call it outside any lane-dependent branch (a
// move compiled under a lane mask reads disabled lanes).
__device__ __forceinline__ float lane_down_or_neg_inf(float x, int k, int lane) {
  const float y = __int_as_float(__builtin_amdgcn_ds_bpermute((lane + k) << 2, __float_as_int(x)));
  return lane + k < 64 ? y : -INFINITY;
}

// Inclusive suffix maximum over the lanes: max of x over lanes >= L.
__device__ __forceinline__ float suffix_max(float x, int lane) {
  x = fmaxf(x, lane_down_or_neg_inf(x, 1, lane));
  x = fmaxf(x, lane_down_or_neg_inf(x, 2, lane));
  x = fmaxf(x, lane_down_or_neg_inf(x, 4, lane));
  x = fmaxf(x, lane_down_or_neg_inf(x, 8, lane));
  x = fmaxf(x, lane_down_or_neg_inf(x, 16, lane));
  return fmaxf(x, lane_down_or_neg_inf(x, 32, lane));
}

// ml_step of every partition of a row at once, for up to 128 partitions: lane
// L holds partitions L and L + 64 (m0 / m1; partitions at or past `parts`
// count as empty).  The running maximum before partition p is the maximum of
// the partitions after it (a suffix maximum), so each lane computes its
// partitions' steps without the chain: the same fmaxf / exp_fast operations
// on the same values as ml_step in order, hence the same bits.
__device__ __forceinline__ void ml_steps_of(float m0, float m1, int parts, int lane, MlStep& s0,
                                            MlStep& s1) {
  const float v0 = lane < parts ? m0 : -INFINITY;
  const float v1 = lane + 64 < parts ? m1 : -INFINITY;
  const float hi = suffix_max(v1, lane);  // max over partitions >= L + 64
  const float hi_all = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(hi)));
  const float lo = fmaxf(suffix_max(v0, lane), hi_all);
  // The maximum of the partitions after p (-inf after the last).
  const float after1 = lane_down_or_neg_inf(hi, 1, lane);
  const float after0 = fmaxf(lane_down_or_neg_inf(lo, 1, lane), lane == 63 ? hi_all : -INFINITY);
  float M0 = after0, M1 = after1;
  s0 = ml_step(v0, M0);
  s1 = ml_step(v1, M1);
}

// One wavefront merges columns [c0, c0 + C) (C a multiple of 4) of the G <= GP
// query heads of a GQA group over all `splits` splits, with the arithmetic of
// lse_merge_kernel: merge weights per head from lse_weights, then
// acc = fma(w_p, partial_p, acc) in split order.  `pg` and `lg` are the
// group's first rows of partials [G][splits][D] and lse [G][splits]; `og` its
// first output row [G][D].
// Lane l owns chunks l, l + 64, ... (kNC of them) of 4 consecutive columns;
// chunk i is head i / (C/4), columns c0 + 4 (i % (C/4)), so one 16-byte load
// per split and chunk.  Batches of kBatch splits are issued at once (kBatch *
// kNC stays below the 63 loads a wavefront can have in flight), before the
// weights are computed.  A head's weights reach the lanes through `wsh`, this
// wavefront's 128 * GP floats of LDS: lse_weights leaves w_p in lane p % 64,
// which writes it to wsh[128 h + p], and each lane reads its head's weights
// four splits at a time.  Loads past the last split read past the buffer
// (zero) and have weight 0, so they leave acc unchanged.  kAux is the cache
// policy of the loads: kCoherentAux for values workgroups on other XCDs wrote.
template <int GP, int kNC, int kBatch, int kAux>
__device__ __forceinline__ void merge_group_chunks(const float* __restrict__ pg,
                                                   const float* __restrict__ lg,
                                                   uint16_t* __restrict__ og, int G, int splits,
                                                   int D, int lanes, int c0, int C,
                                                   float* __restrict__ wsh, int lane) {
  static_assert(kBatch % 4 == 0 && kBatch * kNC <= 48, "batch of loads in flight");
  const int cpr = C / 4;  // chunks per head
  const int bytes = G * splits * D * 4;
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(pg, bytes);
  int hd[kNC], off[kNC];
  bool live[kNC];
  float acc[kNC][4];
#pragma unroll
  for (int i = 0; i < kNC; ++i) {
    const int chunk = lane + 64 * i;
    live[i] = chunk < G * cpr;
    hd[i] = live[i] ? chunk / cpr : 0;
    off[i] = ((hd[i] * splits) * D + c0 + 4 * (chunk % cpr)) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[i][e] = 0.f;
  }
  float x[kBatch][kNC][4];
  auto load = [&](int s0) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
#pragma unroll
      for (int i = 0; i < kNC; ++i)
        buffer_load_f32<4, kAux>(rs, s0 + j < splits ? off[i] + (s0 + j) * D * 4 : bytes,
                                      x[j][i]);
  };
  auto accumulate = [&](int s0) {
#pragma unroll
    for (int j = 0; j < kBatch; j += 4)
#pragma unroll
      for (int i = 0; i < kNC; ++i) {
        // Splits from 128 on do not exist (x = 0 there); their weights are read
        // from splits 124..127, which are finite.
        const int p4 = s0 + j < 128 ? s0 + j : 124;
        const floatx4_t w4 = *reinterpret_cast<const floatx4_t*>(wsh + 128 * hd[i] + p4);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][e] = fmaf(w4[u], x[j + u][i][e], acc[i][e]);
      }
  };
  load(0);
  // Every head's LSE loads go out with the first batch (rows past the group
  // read as empty), so all of them arrive in one round trip.
  float la[GP], lc[GP];
#pragma unroll
  for (int h = 0; h < GP; ++h)
    lse_load<kAux>(lg + int64_t(h < G ? h : 0) * splits, h < G ? splits * 4 : 0, lane, la[h],
                        lc[h]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int h = 0; h < GP; ++h) {
    if (h >= G) break;
    float w0, w1;
    lse_weights_of(la[h], lc[h], splits, lanes, lane, w0, w1);
    wsh[128 * h + lane] = w0;
    wsh[128 * h + 64 + lane] = w1;
  }
  accumulate(0);
  for (int s0 = kBatch; s0 < splits; s0 += kBatch) {
    load(s0);
    accumulate(s0);
  }
#pragma unroll
  for (int i = 0; i < kNC; ++i) {
    if (!live[i]) continue;
    const int chunk = lane + 64 * i;
    uint16_t* dst = og + int64_t(hd[i]) * D + c0 + 4 * (chunk % cpr);
    *reinterpret_cast<u32x2_t*>(dst) =
        u32x2_t{bf16_bits(acc[i][0]) | (bf16_bits(acc[i][1]) << 16),
                bf16_bits(acc[i][2]) | (bf16_bits(acc[i][3]) << 16)};
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
// each 16-token group, which for two groups g, g+1 side by side is the A
// layout of v_mfma_f32_16x16x32_bf16
// (k = 8*(L/16) + e <-> token 16g + 4*(L/16) + e for e < 4, 16(g+1) +
// 4*(L/16) + e-4 above).  The B operand needs V columns (4 consecutive tokens
// of one d per lane).  V rows therefore go to LDS by buffer_load ... lds (no
// registers; lane l of a copy fills bytes 16l .. 16l+15 of its 1 KiB, and
// reads past the buffer write zeros), with the 16-byte pieces of each row
// swizzled (vswz) so that the transposed reads hit distinct banks, and are
// read with
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
  static constexpr int kPieces = D / 8;                      // 16-byte pieces per V row
  static constexpr int kPitch = 16 * kPieces;                // bytes per V row in LDS
  static constexpr int kDma = kTW * kPitch / 1024;           // 1 KiB copies per wavefront
  static constexpr int kSlot = 1024 * kDma;                  // LDS bytes of a wavefront's rows
  static_assert(kNG >= 1 && kCH >= 1 && kTW * kPitch % 1024 == 0, "geometry");
};

// V rows sit in LDS unpadded (kPitch = 2D bytes), with the 16-byte pieces of
// each row permuted: piece p of row r is stored at position p ^ vswz(r).  The
// LDS serves 32 lanes of a ds_read_b64_tr_b16 per clock, 256 bytes over 64
// four-byte banks; each lane's 8 bytes are two pieces' halves of one row, and
// each row's 4 lanes read two adjacent pieces (32 bytes).  The 32 lanes must
// therefore land on 8 distinct 32-byte bank groups.  The kernels split P V by
// output columns: lanes 0-15 read rows 0-3 of a 32-row k-step and lanes 16-31
// rows 8-11 (rows 4-7 and 12-15 in the second read of the step, which takes
// the same swizzle).  Rows of 2D >= 256 bytes start on bank 0, so the swizzle
// alone spreads them: bits 0-1 of the row pick one of 4 pairs of pieces, and
// bit 3 one of two 128-byte halves.  Rows of 128 bytes (D = 64) alternate
// between the two halves by their own address (bit 0), so the swizzle spreads
// the rows of one half over its 4 pairs of pieces.  (A swizzle by r mod 4
// alone left a 2-way conflict on every read.)
//
// kRows (D = 64 only): the reads of P V by rows (each compute wavefront
// multiplying its own rows by all 64 columns) take rows 4c .. 4c + 3 of a
// 16-row group in lanes 16c .. 16c + 15 of each 32-lane half, so rows 0-7 of
// a group share a clock instead of rows 0-3 and 8-11: bit 2 of the row picks
// the pair instead of bit 3.
template <int D, bool kRows = false>
__device__ __forceinline__ int vswz(int row) {
  static_assert(!kRows || D == 64, "row-wise P V swizzle at D = 64 only");
  if constexpr (D >= 128)
    return 2 * (row & 3) + 8 * ((row >> 3) & 1);
  else if constexpr (kRows)
    return 2 * (((row >> 1) & 1) | (((row >> 2) & 1) << 1));
  else
    return 2 * (((row >> 1) & 1) | (((row >> 3) & 1) << 1));
}

// Element offset (tile-relative) of tile row R: token R / H of the
// workgroup's kv head R % H, for H kv heads per workgroup (their rows of a
// token are adjacent; RS = Hkv * D elements per token).
template <int D, int H>
__device__ __forceinline__ int tile_row_elems(int R, int RS) {
  return (R / H) * RS + (R % H) * D;
}

// Source byte offset (tile-relative) of the 16 bytes that DMA copy i of
// wavefront w places at LDS position 16 * (64 i + lane) of its rows.
template <int D, int GP, int H = 1, bool kRows = false>
__device__ __forceinline__ int v_copy_offset(int i, int lane, int w, int RS) {
  using C = Matched<D, GP>;
  const int slot = 64 * i + lane;
  const int row = slot / C::kPieces, pos = slot % C::kPieces;
  return (tile_row_elems<D, H>(w * C::kTW + row, RS) + 8 * (pos ^ vswz<D, kRows>(row))) * 2;
}

// Byte offset within a V row of this lane's 8 bytes of a transposed read of
// the 16 columns from col0 (a multiple of 16): lane l % 4 = b reads columns
// col0 + 4b .. +3 of a row whose index within its 16-row group is `row`.
template <int D, bool kRows = false>
__device__ __forceinline__ int v_read_offset(int col0, int lane, int row) {
  const int b = lane & 3;
  return 16 * (((col0 >> 3) + (b >> 1)) ^ vswz<D, kRows>(row)) + 8 * (b & 1);
}

// K rows staged in LDS by loader wavefronts (cols_loader_kernel): row r of a
// tile holds its 16-byte piece p at position p ^ kswz(r).  A compute
// wavefront's ds_read_b128 reads one piece from each of 16 consecutive rows,
// and 16 lanes are served per clock (256 bytes over 64 four-byte banks), so
// the 16 pieces must fall on distinct 16-byte bank groups: rows of 2D >= 256
// bytes start on bank 0 and the XOR with r & 15 spreads them; 128-byte rows
// (D = 64) alternate halves by address and the XOR with (r >> 1) & 7 spreads
// each half.  The XOR keeps aligned groups of 8 pieces together, so eight
// consecutive lanes of a loader copy still read one 128-byte line.
template <int D>
__device__ __forceinline__ int kswz(int row) {
  return D >= 128 ? (row & 15) : ((row >> 1) & 7);
}

template <int D, int GP>
struct KTile {
  u32x4_t k[Matched<D, GP>::kNG][Matched<D, GP>::kCH];
};

// K rows are fetched as whole 128-byte lines and rearranged into the MFMA
// A-operand layout in registers.  A load in the operand layout itself (lane
// 16g + r: row r, 16 bytes at 16g of a 64-byte piece) covers 16 rows x 64
// bytes, half lines whose consecutive lanes address different rows, and one
// CU streams such loads at about half the rate of loads whose eight
// consecutive lanes cover one line (38 vs 72 GB/s per CU, measured on
// MI355X).  So load (h, sh) of a 16-row group gives lane S = 8k + p row
// 8sh + k, 16-byte chunk c(S) of line h, with c = p for S < 32 and the
// chunks rotated by two in the upper half, c = (p - 2) mod 8 for S >= 32
// (kline_offset; each 8 consecutive lanes still cover one line).  The bank-
// masked DPP moves within 16-lane rows (banks 1 and 3 are the lanes p >= 4)
// pair chunks four apart:
//   u = load 0 on lanes p < 4, load 1 from lane S - 4 on lanes p >= 4;
//   v = load 0 from lane S + 4 on lanes p < 4, load 1 on lanes p >= 4,
// and in the upper half, where the rotation puts the higher chunk of a pair
// first on lanes with p & 2 = 0, u and v are exchanged there.  Lane S then
// holds chunks c' and c' + 4 of one row, c' < 4; one ds_bpermute per dword
// fetches lane 16g + r's chunks g and g + 4 of row r from lane
// 8 (r mod 8) + 4 [r >= 8] + (r mod 8 < 4 ? g : (g + 2) mod 4) (kline_source).
// The rotation makes the 32 source lanes of each half-wavefront distinct
// modulo 32: without it rows k and k + 4 sat on lanes 32 apart and every
// ds_bpermute read had 2-way bank conflicts.
// The single-tile kernel loads its one tile this way (all of it in flight at
// once, so the load rate is what counts).  The multi-tile loop keeps loads in
// the operand layout: there the rearrangement lengthens every tile's chain
// and one streaming workgroup slowed from 57 to 41 GB/s.
__device__ __forceinline__ int kline_offset(int lane, int RS) {
  const int p = lane & 7;
  const int chunk = lane >= 32 ? ((p - 2) & 7) : p;
  return ((lane >> 3) * RS + 8 * chunk) * 2;
}
__device__ __forceinline__ int kline_source(int lane) {
  const int r = lane & 15, g = lane >> 4, k = r & 7;
  return 4 * (8 * k + (r >= 8 ? 4 : 0) + (k >= 4 ? ((g + 2) & 3) : g));
}
__device__ __forceinline__ void lines_to_mfma(u32x4_t& a, u32x4_t& b, int src, bool exchange) {
  u32x4_t ra, rb;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int u = __builtin_amdgcn_update_dpp(int(a[e]), int(b[e]), 0x114, 0xf, 0xa, false);
    const int v = __builtin_amdgcn_update_dpp(int(b[e]), int(a[e]), 0x104, 0xf, 0x5, false);
    ra[e] = unsigned(__builtin_amdgcn_ds_bpermute(src, exchange ? v : u));
    rb[e] = unsigned(__builtin_amdgcn_ds_bpermute(src, exchange ? u : v));
  }
  a = ra;
  b = rb;
}

template <int D, int GP>
__device__ __forceinline__ void ktile_to_mfma(KTile<D, GP>& R, int lane) {
  const int src = kline_source(lane);
  const bool exchange = lane >= 32 && !(lane & 2);
#pragma unroll
  for (int g = 0; g < Matched<D, GP>::kNG; ++g)
#pragma unroll
    for (int h = 0; h < Matched<D, GP>::kCH / 2; ++h)
      lines_to_mfma(R.k[g][2 * h], R.k[g][2 * h + 1], src, exchange);
}

typedef short short4_t __attribute__((ext_vector_type(4)));

// 16 bytes at byte offset `off` of a buffer (zero past its end).
__device__ __forceinline__ u32x4_t buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int off) {
  const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
  return t;
}

// The K rows of a wavefront's share of a tile, as whole-line loads (rows
// 16g + 8sh + S/8 from `kl`, the lane's kline_offset from the share's first
// row); ktile_to_mfma then rearranges them for QK.
template <int D, int GP>
__device__ __forceinline__ void ktile_load(KTile<D, GP>& R, __amdgpu_buffer_rsrc_t rsrc, int kl,
                                           int RS) {
#pragma unroll
  for (int g = 0; g < Matched<D, GP>::kNG; ++g)
#pragma unroll
    for (int h = 0; h < Matched<D, GP>::kCH / 2; ++h) {
      R.k[g][2 * h] = buffer_load16(rsrc, kl + (32 * g) * RS + 128 * h);
      R.k[g][2 * h + 1] = buffer_load16(rsrc, kl + (32 * g + 16) * RS + 128 * h);
    }
}

// Four bf16 of one column, transposed out of LDS (see above).  `p` points
// into a __shared__ array; the LDS address-space casts live in these helpers
// so that kernel bodies only handle ordinary pointers.
__device__ __forceinline__ short4_t lds_read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4_t*)(const_cast<char*>(p)));
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const char*)(p)));
}

// ds_read_b64_tr_b16 at LDS byte address base + OFF, issued from inline asm.
// The compiler does not see an LDS read, so it neither adds waits for LDS
// copies (buffer_load ... lds) into the same array nor waits for the result:
// the caller orders the read after the copies it needs and passes the results
// through lds_settle before using them.
template <int OFF>
__device__ __forceinline__ short4_t lds_read_tr_at(uint32_t base) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  short4_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(base), "i"(OFF));
  return r;
}

// 16 bytes at an LDS byte address (ds_read_b128), issued from inline asm as
// lds_read_tr_at is; the results pass through lds_wait before use.
__device__ __forceinline__ u32x4_t lds_read16_at(uint32_t addr) {
  u32x4_t r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

// 4 bytes at an LDS byte address (ds_read_b32), from inline asm like
// lds_read16_at; the result passes through lds_wait before use.
__device__ __forceinline__ uint32_t lds_read4_at(uint32_t addr) {
  uint32_t r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

// Waits for every LDS read of this wavefront and makes the uses of x follow.
template <int N>
__device__ __forceinline__ void lds_wait(u32x4_t (&x)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(x[i]));
}

// s_waitcnt vmcnt(N): at most N vector-memory loads of this wavefront remain
// outstanding (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// s_waitcnt vmcnt(0): every vector-memory load AND store this wavefront has
// issued has completed (on gfx9-family GPUs stores are counted in vmcnt too).
// A device-scope (sc1) store has then been written through to the coherence
// point, so a workgroup on another XCD that reads the line with a
// device-scope load sees it.  A barrier or a workgroup-scope fence does not
// wait for other wavefronts' stores: each wavefront waits for its own.
__device__ __forceinline__ void wait_memory() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Waits for every outstanding LDS read (lgkmcnt(0)) and makes the values
// depend on that wait, so no use of them is scheduled before it.
template <int N>
__device__ __forceinline__ void lds_settle(short4_t (&a)[N], short4_t (&b)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(a[i]), "+v"(b[i]));
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

// ------------------------------------------------------------- batch order
// Which sequence the workgroups of grid row z serve.  Every (split, kv head,
// sequence) item computes the same values whichever workgroup runs it, so a
// launch may hand the grid rows to the sequences in any order; taking them by
// length evens out the work per CU when the grid runs in several rounds (one
// workgroup per CU), since the longest items then start first.  `order`
// (chosen by the launcher from the grid and the CU count):
//   < 0   row z serves sequence z;
//   0     row z serves the sequence of length rank z.
// Ranks order the lengths decreasing, ties by increasing index, so they are a
// permutation of [0, B).
constexpr int kMaxOrderedBatch = 256;
static_assert(kMaxOrderedBatch == kThreads, "one thread per sequence");

struct OrderedSequence {
  int b, length;
};

// Requires order == 0, 2 <= B <= kMaxOrderedBatch, blockDim.x >= kThreads and
// every thread of the workgroup; `slens` holds kMaxOrderedBatch + 4 ints of LDS,
// 16-byte aligned.  One load of the lengths, then thread t counts the
// sequences ranked before sequence t; the one of rank z publishes its index.
__device__ __forceinline__ OrderedSequence ordered_sequence(const int32_t* __restrict__ lengths,
                                                            int B, int z, int order,
                                                            int* __restrict__ slens) {
  const int tid = threadIdx.x;
  // Entries past B hold INT_MIN: never longer, and a tie only with an index >= B.
  const int len = tid < B ? lengths[tid] : INT32_MIN;
  if (tid < kMaxOrderedBatch) slens[tid] = len;
  if (tid == 0) slens[kMaxOrderedBatch] = z;  // overwritten below by the one match
  __syncthreads();
  if (tid < B) {
    int rank = 0;
    const int4* s4 = reinterpret_cast<const int4*>(slens);
    for (int u = 0; u < B; u += 4) {
      const int4 x = s4[u >> 2];
      rank += int(x.x > len) + int(x.x == len && u < tid);
      rank += int(x.y > len) + int(x.y == len && u + 1 < tid);
      rank += int(x.z > len) + int(x.z == len && u + 2 < tid);
      rank += int(x.w > len) + int(x.w == len && u + 3 < tid);
    }
    if (rank == z) slens[kMaxOrderedBatch] = tid;
  }
  __syncthreads();
  const int b = __builtin_amdgcn_readfirstlane(slens[kMaxOrderedBatch]);
  return {b, __builtin_amdgcn_readfirstlane(slens[b])};
}

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

}  // namespace pdk

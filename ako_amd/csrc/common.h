// Shared device helpers for the gfx950 (CDNA4) streaming kernels.
//
// Storage types are float, _Float16 and __bf16. Every kernel widens to fp32,
// computes, and narrows with round-to-nearest-even (v_cvt_f16_f32 and, on
// gfx950, v_cvt_pk_bf16_f32). Global memory is moved in 16-byte packets
// (global_load_dwordx4 / global_store_dwordx4), optionally with the
// non-temporal hint for data that is touched exactly once.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fastdiv.h"

namespace ako {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Division by a launch-invariant divisor (FastDiv, built on the host by
// make_fastdiv): a multiply-high and two shifts, exact for every 32-bit
// unsigned dividend, instead of the reciprocal-and-correct sequence of a
// runtime division on the path to a wavefront's first load.
__device__ __forceinline__ unsigned fast_div(unsigned n, const FastDiv& f) {
  const unsigned t = __umulhi(f.m, n);
  return (t + ((n - t) >> f.s1)) >> f.s2;
}

// ---- scalar conversions -------------------------------------------------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) {
  return static_cast<_Float16>(v);
}
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) {
  return static_cast<__bf16>(v);
}

// ---- raw packets of 2..16 bytes --------------------------------------------
template <int BYTES> struct RawOf;
template <> struct RawOf<16> { using type = u32x4; };
template <> struct RawOf<8> { using type = u32x2; };
template <> struct RawOf<4> { using type = unsigned int; };
template <> struct RawOf<2> { using type = unsigned short; };

// N elements of T viewed as one register packet (N * sizeof(T) <= 16 bytes).
template <typename T, int N>
union Pack {
  static constexpr int kBytes = N * static_cast<int>(sizeof(T));
  using raw_t = typename RawOf<kBytes>::type;
  raw_t raw;
  T e[N];
};

template <bool NT, typename R>
__device__ __forceinline__ R load_raw(const R* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}

template <bool NT, typename R>
__device__ __forceinline__ void store_raw(R* p, R v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

template <typename T, int N, bool NT = false>
__device__ __forceinline__ Pack<T, N> load_pack(const T* p) {
  Pack<T, N> pk;
  pk.raw = load_raw<NT>(reinterpret_cast<const typename Pack<T, N>::raw_t*>(p));
  return pk;
}

template <typename T, int N, bool NT = false>
__device__ __forceinline__ void store_pack(T* p, const Pack<T, N>& pk) {
  store_raw<NT>(reinterpret_cast<typename Pack<T, N>::raw_t*>(p), pk.raw);
}

// N consecutive elements of T (any N that splits into <=16-byte packets),
// widened to fp32. p must be aligned to min(16, N * sizeof(T)) bytes.
template <typename T, int N, bool NT = false>
__device__ __forceinline__ void load_f32(const T* p, float (&out)[N]) {
  constexpr int kPer = (16 / static_cast<int>(sizeof(T))) < N ? (16 / static_cast<int>(sizeof(T))) : N;
  static_assert(N % kPer == 0, "pack split");
#pragma unroll
  for (int c = 0; c < N / kPer; ++c) {
    Pack<T, kPer> pk = load_pack<T, kPer, NT>(p + c * kPer);
#pragma unroll
    for (int i = 0; i < kPer; ++i) out[c * kPer + i] = to_f32(pk.e[i]);
  }
}

// ---- sum of squares of one packet -------------------------------------------
// acc + sum of e^2 over the packet's elements. bf16 packets go two elements
// per v_dot2c_f32_bf16: products of bf16 values are exact in fp32, so only the
// accumulation order differs from a chain of fp32 FMAs, and one instruction
// replaces two shift/mask widenings and two FMAs (measured +1-1.4% on the
// widest bf16 rows). fp16 already widens inside v_fma_mix_f32 and gains
// nothing from v_dot2, so it keeps the FMA chain.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <typename T, int N>
__device__ __forceinline__ float sumsq_add(const Pack<T, N>& p, float acc) {
  if constexpr (__is_same(T, __bf16) && Pack<T, N>::kBytes == 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x2 h = __builtin_bit_cast(bf16x2, static_cast<unsigned>(p.raw[i]));
      acc = __builtin_amdgcn_fdot2_f32_bf16(h, h, acc, false);
    }
    return acc;
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float f = to_f32(p.e[e]);
      acc = __builtin_fmaf(f, f, acc);
    }
    return acc;
  }
}

// ---- wavefront reduction ----------------------------------------------------
// Butterfly all-reduce over 64 lanes: DPP quad permutes and row mirrors inside
// each 16-lane row (no LDS traffic), then two ds_bpermute steps across rows.
// Every step adds a lane to its partner symmetrically, so all 64 lanes end
// with the bitwise-identical total.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp_mov<0x141>(v);  // row_half_mirror: the other quad of each 8 lanes
  v += dpp_mov<0x140>(v);  // row_mirror: the other half of each 16-lane row
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// ---- workgroup order over the XCDs ------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on
// XCD b % 8). block_order hands each XCD runs of `chunk` consecutive blocks:
// workgroup b = 8 i + x takes block c * 8 chunk + x * chunk + j for
// i = c * chunk + j, so the XCDs walk 8 separate runs instead of interleaving
// block by block. chunk <= 1 is the identity; the last, partial round of runs
// is split evenly the same way and the n % 8 trailing blocks keep their own
// index, which keeps the map a bijection on [0, n).
struct XcdRuns {
  unsigned chunk;    // consecutive blocks per run; <= 1 keeps block order
  FastDiv by_chunk;  // divides by max(chunk, 1)
};

inline XcdRuns make_xcd_runs(unsigned chunk) { return XcdRuns{chunk, make_fastdiv(chunk > 1 ? chunk : 1)}; }

// The two divisions by the run length are multiply-shifts (a runtime
// division costs a reciprocal-and-correct sequence on the path to a new
// workgroup's first load). Block order (every decode-sized launch) returns
// before any of it: computing the runs anyway, without the branch, made
// one-row launches 0.06-0.2 us slower.
__device__ __forceinline__ unsigned block_order(unsigned b, unsigned n, const XcdRuns& r) {
  const unsigned q = n / 8;
  if (r.chunk <= 1 || b >= 8 * q) return b;
  const unsigned x = b % 8, i = b / 8;
  const unsigned full = fast_div(q, r.by_chunk);
  const unsigned c = fast_div(i, r.by_chunk), j = i - c * r.chunk;
  if (c < full) return c * 8 * r.chunk + x * r.chunk + j;
  const unsigned rest = q - full * r.chunk;
  return full * 8 * r.chunk + x * rest + (i - full * r.chunk);
}

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace ako

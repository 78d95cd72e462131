// SwiGLU activation y = silu(gate) * up for gfx950.
//
// swiglu_flat - the three tensors are one dense block each: a 1-D stream of
//   16-byte packets. Each lane owns U packets spaced BLOCK apart inside its
//   workgroup's tile (every wavefront-wide load covers 1 KiB contiguous), and
//   issues all 2*U loads before computing. Elements after the last full
//   packet are handled by the first lanes of workgroup 0.
// swiglu_rows - strided rows (or any alignment when E = 1): a workgroup owns a
//   (row, column-tile) pair, block index split on the host-visible grid.
//
// Math: silu(g) * u = (g / (1 + e^-g)) * u in fp32 (the form of the
// reference's fp32 silu), rounded to the storage dtype. Half-precision
// outputs use the hardware transcendental path: e^-g = v_exp_f32(-g*log2 e)
// and the division as g * v_rcp_f32(1 + e^-g), each accurate to about one
// fp32 ulp, i.e. ~2^-13 of a half-precision ulp; this keeps the kernel under
// the VALU budget of an 8 TB/s stream (about 14 VALU cycles per element
// instead of ~30 for the IEEE sequences). fp32 outputs use the correctly
// rounded division and the libm-accurate expf.

#include <algorithm>

#include "common.h"
#include "launch.h"

namespace ako {

SwigluTuning g_swiglu_tuning;

template <typename T>
__device__ __forceinline__ float silu_mul(float g, float u) {
  if constexpr (sizeof(T) == 4) {
    return (g / (1.0f + expf(-g))) * u;
  } else {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    // v_rcp_f32 flushes a subnormal result, so 1 / (1 + e) is 0 once
    // 1 + e > 2^126 (g < -87.3) although g / (1 + e) is still a normal number
    // down to g = -88.7, where exp overflows. Above 2^64 the denominator is
    // scaled down by 2^64 before the reciprocal and the quotient back after
    // it, both exact.
    const float d = 1.0f + e;
    const bool big = d > 0x1p64f;
    const float s = g * __builtin_amdgcn_rcpf(big ? d * 0x1p-64f : d);
    return (big ? s * 0x1p-64f : s) * u;
  }
}

template <typename T, int U, int BLOCK>
__global__ __launch_bounds__(BLOCK) void swiglu_flat(const T* __restrict__ g,
                                                     const T* __restrict__ u, T* __restrict__ y,
                                                     int64_t first_packet, int64_t npackets,
                                                     int64_t nelems, XcdRuns runs) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  using P = Pack<T, E>;
  const int64_t base = first_packet +
                       static_cast<int64_t>(block_order(blockIdx.x, gridDim.x, runs)) * (BLOCK * U) + threadIdx.x;
  P gv[U], uv[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t vi = base + k * BLOCK;
    if (vi < npackets) {
      gv[k] = load_pack<T, E, true>(g + vi * E);
      uv[k] = load_pack<T, E, true>(u + vi * E);
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t vi = base + k * BLOCK;
    if (vi < npackets) {
      P o;
#pragma unroll
      for (int e = 0; e < E; ++e) o.e[e] = from_f32<T>(silu_mul<T>(to_f32(gv[k].e[e]), to_f32(uv[k].e[e])));
      store_pack<T, E, true>(y + vi * E, o);
    }
  }
  if (first_packet == 0 && blockIdx.x == 0) {
    const int64_t i = npackets * E + threadIdx.x;
    if (i < nelems) y[i] = from_f32<T>(silu_mul<T>(to_f32(g[i]), to_f32(u[i])));
  }
}

template <typename T, int E, int U, int BLOCK>
__global__ __launch_bounds__(BLOCK) void swiglu_rows(const T* __restrict__ g,
                                                     const T* __restrict__ u, T* __restrict__ y,
                                                     int64_t row0, int n, int tiles, int64_t sg,
                                                     int64_t su, int64_t sy) {
  using P = Pack<T, E>;
  const int64_t row = row0 + blockIdx.x / tiles;
  const int tile = blockIdx.x % tiles;
  const int npk = n / E;
  const T* gr = g + row * sg;
  const T* ur = u + row * su;
  T* yr = y + row * sy;
  const int base = tile * (BLOCK * U) + threadIdx.x;
  P gv[U], uv[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int vi = base + k * BLOCK;
    if (vi < npk) {
      gv[k] = load_pack<T, E, true>(gr + vi * E);
      uv[k] = load_pack<T, E, true>(ur + vi * E);
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int vi = base + k * BLOCK;
    if (vi < npk) {
      P o;
#pragma unroll
      for (int e = 0; e < E; ++e) o.e[e] = from_f32<T>(silu_mul<T>(to_f32(gv[k].e[e]), to_f32(uv[k].e[e])));
      store_pack<T, E, true>(yr + vi * E, o);
    }
  }
  if (tile == 0) {
    const int i = npk * E + threadIdx.x;
    if (i < n) yr[i] = from_f32<T>(silu_mul<T>(to_f32(gr[i]), to_f32(ur[i])));
  }
}

namespace {

constexpr int kBlock = 256;
constexpr int64_t kMaxBlocksPerLaunch = int64_t(1) << 22;  // grid work-items stay < 2^32

template <typename T, int U>
hipError_t run_flat(const SwigluArgs& a, hipStream_t stream) {
  constexpr int E = 16 / sizeof(T);
  const int64_t nelems = a.rows * a.n;
  const int64_t npk = nelems / E;
  const int64_t per_block = int64_t(kBlock) * U;
  const int64_t blocks = std::max<int64_t>(1, ceil_div(npk, per_block));
  // Launches of kRunsMinBlocks to kRunsMaxBlocks - 1 workgroups hand them to
  // the XCDs in runs of kRun; smaller ones (decode) and larger ones keep
  // block order. Against block order, bf16 x 14336, 4-6 buffer placements
  // (random spacers between the input copies, interleaved back-to-back
  // timings) on each of five MI355X boxes: M = 4096 +0.7 to +2.5 points of
  // peak (box means), M = 512-1024 +0.3 to +1.2, M = 8192 +1.25 (one box);
  // M = 16384 (114688 workgroups) -0.55 to +0.9 by box, +0.2 on average;
  // M = 256 (1792 workgroups) -0.3. Key 2 overrides (1 = block order).
  constexpr int64_t kRunsMinBlocks = 2048;
  constexpr int64_t kRunsMaxBlocks = 65536;
  constexpr unsigned kRun = 4;
  const int forced = g_swiglu_tuning.xcd_chunk;
  for (int64_t b0 = 0; b0 < blocks; b0 += kMaxBlocksPerLaunch) {
    const int64_t nb = std::min(kMaxBlocksPerLaunch, blocks - b0);
    const bool runs_by_default = nb >= kRunsMinBlocks && nb < kRunsMaxBlocks;
    const unsigned chunk = forced > 0 ? static_cast<unsigned>(forced) : (runs_by_default ? kRun : 1u);
    const XcdRuns runs = make_xcd_runs(chunk);
    AKO_LAUNCH((swiglu_flat<T, U, kBlock>), dim3(static_cast<unsigned>(nb)), dim3(kBlock), 0,
               stream, static_cast<const T*>(a.g), static_cast<const T*>(a.u),
               static_cast<T*>(a.y), b0 * per_block, npk, nelems, runs);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

template <typename T, int E, int U>
hipError_t run_rows(const SwigluArgs& a, hipStream_t stream) {
  const int n = static_cast<int>(a.n);
  const int tiles = static_cast<int>(std::max<int64_t>(1, ceil_div(n / E, int64_t(kBlock) * U)));
  const int64_t rows_per_launch = std::max<int64_t>(1, kMaxBlocksPerLaunch / tiles);
  for (int64_t r0 = 0; r0 < a.rows; r0 += rows_per_launch) {
    const int64_t nr = std::min(rows_per_launch, a.rows - r0);
    AKO_LAUNCH((swiglu_rows<T, E, U, kBlock>), dim3(static_cast<unsigned>(nr * tiles)),
               dim3(kBlock), 0, stream, static_cast<const T*>(a.g),
               static_cast<const T*>(a.u), static_cast<T*>(a.y), r0, n, tiles, a.sg, a.su,
               a.sy);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

template <typename T>
hipError_t run_typed(const SwigluArgs& a, hipStream_t stream) {
  constexpr int E = 16 / sizeof(T);
  // One packet per lane (measured on MI355X: 6.57 TB/s at U=1 against
  // 6.12 TB/s at U=4 for 16384 x 14336 bf16; graph-replayed decode calls at
  // M = 1 / 16 / 256 take 1.80 / 1.79 / 4.35 us at U=1 against 1.88 / 2.00 /
  // 4.75 us at U=2).
  int unroll = g_swiglu_tuning.vecs_per_thread;
  if (unroll <= 0) unroll = 1;
  if (!a.vector_ok) return run_rows<T, 1, 4>(a, stream);
  if (a.contiguous) {
    if (unroll <= 1) return run_flat<T, 1>(a, stream);
    if (unroll <= 2) return run_flat<T, 2>(a, stream);
    if (unroll <= 4) return run_flat<T, 4>(a, stream);
    return run_flat<T, 8>(a, stream);
  }
  return unroll <= 2 ? run_rows<T, E, 2>(a, stream) : run_rows<T, E, 4>(a, stream);
}

}  // namespace

hipError_t launch_swiglu(const SwigluArgs& a, hipStream_t stream) {
  switch (a.dtype) {
    case kF32: return run_typed<float>(a, stream);
    case kF16: return run_typed<_Float16>(a, stream);
    case kBF16: return run_typed<__bf16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ako

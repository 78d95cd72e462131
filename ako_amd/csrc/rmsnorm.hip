// RMSNorm and residual-add + RMSNorm for gfx950.
//
// Three kernels:
//
// rmsnorm_reg  - the row lives in registers. A row is owned by WPR wavefronts
//   (64 * WPR lanes); lane t of the row holds the 16-byte packets
//   t, t + 64*WPR, t + 2*64*WPR, ... (VPT of them), so every wavefront-wide
//   load instruction covers 1 KiB of contiguous memory. HBM is touched once
//   per element: x (and the residual) are read once, y (and the new
//   residual) written once, all with the non-temporal hint; the weight row
//   is re-read by every row and stays in L2. The sum of squares is reduced
//   in fp32 with DPP inside the wavefront and, when WPR > 1, through WPR
//   floats of LDS. Small rows pack RPB rows into one workgroup (the decode
//   shapes: 1 or 32 rows). A lane issues every load of a group of packets
//   before consuming any of them, so its memory latency is paid once per
//   group instead of once per packet. Wide rows are handed to the 8 XCDs in
//   runs of consecutive rows (block_order) rather than row by row.
//
// rmsnorm_pipe - rmsnorm_reg's row layout in a persistent, software-pipelined
//   grid: each workgroup walks a sequence of rows and issues the next row's
//   loads before it reduces and writes the current one. Taken by launches of
//   many full rows of at most 16 KiB of input at one packet per lane.
//
// rmsnorm_stream - any width, any alignment (E = 1 scalar packets when the
//   rows are not 16-byte aligned). One 256-lane workgroup per row, two passes
//   over global memory: the first accumulates the sum of squares (and writes
//   the rounded residual sum), the second re-reads and normalises. Used for
//   rows wider than the register budget (> 65536 half-precision elements)
//   and for misaligned rows.
//
// Numerics follow the unfused reference (ako/ops/rmsnorm_ref.py:8-50):
//   var  = sum(x^2) * (1/H)          (fp32; 1/H rounded to fp32 on the host)
//   rstd = rsqrt(var + eps)
//   y    = to_T((x * rstd) * w)      (two rounded fp32 multiplies, this order)
// and for the residual variant s = to_T(x + r) is normalised, as the
// reference adds in the storage dtype before normalising.

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace ako {

RmsTuning g_rms_tuning;

// E elements of the weight row held as raw packets (one 16-byte packet, or
// two when the weight is fp32 and the input half precision).
template <typename W, int E>
struct WeightPacket {
  static constexpr int kPer = (16 / static_cast<int>(sizeof(W))) < E ? (16 / static_cast<int>(sizeof(W))) : E;
  Pack<W, kPer> part[E / kPer];
  __device__ __forceinline__ void load(const W* p) {
#pragma unroll
    for (int c = 0; c < E / kPer; ++c) part[c] = load_pack<W, kPer>(p + c * kPer);
  }
  __device__ __forceinline__ float operator[](int e) const { return to_f32(part[e / kPer].e[e % kPer]); }
};

// Write-through stores: a raw buffer store with the sc1 and nt bits, on a
// resource built from the row's base address (uniform across the
// wavefront) and covering exactly the row, so a store past its end would be
// dropped by the hardware. The data go through the XCD's L2 to memory
// instead of staying there as dirty lines until the end of the kernel.
// Measured on MI355X, 16384 rows of 16384 half elements, three alternating
// runs of two builds, back to back: plain rows +1.5 (fp16) and +2.7 (bf16)
// points of peak, residual fp16 rows +0.8 with one packet per load group
// (with whole groups, -1.6), residual bf16 unchanged; rows of 8 KiB or less
// were slower (pipelined 16 KiB-input rows: 82-87% down to 69-70%), so by
// default only the (16, 2) shape uses it (key 12 = 2 selects it on (16, 1)
// rows too).
constexpr int kRawBufferWord3 = 0x00020000;  // raw (untyped) access, gfx9 CDNA layout
constexpr int kStoreSc1Nt = 18;              // cache policy bits: nt (2) | sc1 (16)

template <typename T, int E>
__device__ __forceinline__ void store_write_through(T* row_base, int row_bytes, int elem, const Pack<T, E>& pk) {
  static_assert(E * sizeof(T) == 16, "whole 16-byte packets");
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(row_base, 0, row_bytes, kRawBufferWord3);
  __builtin_amdgcn_raw_buffer_store_b128(pk.raw, r, elem * static_cast<int>(sizeof(T)), 0, kStoreSc1Nt);
}

template <typename T, typename W, int WPR, int VPT, int RPB, bool RES, bool EW, bool SPLIT = false,
          bool WT = false>
__global__ __launch_bounds__(kWave* WPR* RPB) void rmsnorm_reg(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    T* __restrict__ y, T* __restrict__ rout, int64_t row0, int64_t rows, int hidden, int64_t sx,
    int64_t sr, int64_t sy, int64_t srout, float inv_h, float eps, XcdRuns runs) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements per packet
  constexpr int TPR = kWave * WPR;                     // lanes per row
  // Packets are processed in groups: every load of a group is issued before
  // the first of them is consumed, so a lane's memory latency is paid once
  // per group rather than once per packet. Groups stay small enough that x,
  // the residual and the prefetched weights fit in registers. SPLIT makes
  // every packet its own group (the next packet's loads are issued after the
  // previous one is added, stored and squared).
  constexpr int G = SPLIT ? 1 : (VPT <= 4 ? VPT : (VPT <= 8 ? 4 : 2));
  static_assert(VPT % G == 0, "VPT must be a multiple of the group size");
  // With few packets per lane the first weight group is fetched before the
  // reduction; with many, registers are kept for x and weights come per group.
  // EW (early weights, decode-sized launches) issues the first weight group in
  // the same batch as the row's own loads: a launch of a few rows is one
  // dependent chain, and a norm weight that the rest of a model step has
  // evicted then costs one HBM round trip instead of a second one after x.
  static_assert(!EW || VPT <= 4, "early weights need the first group's weights in registers");
  constexpr bool kPrefetchW = VPT <= 4;
  using P = Pack<T, E>;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row_in_block = wave / WPR;
  const int wave_in_row = wave - row_in_block * WPR;
  const int t = wave_in_row * kWave + lane;
  const int64_t row = row0 + static_cast<int64_t>(block_order(blockIdx.x, gridDim.x, runs)) * RPB + row_in_block;
  const bool active = row < rows;
  const int nvec = hidden / E;
  const int tail = hidden - nvec * E;

  const T* xr = x + row * sx;
  T* yr = y + row * sy;

  P v[VPT];
  WeightPacket<W, E> wv[G];
  float ss = 0.f;
#pragma unroll
  for (int g0 = 0; g0 < VPT; g0 += G) {
    [[maybe_unused]] P rv[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int vi = t + (g0 + k) * TPR;
      if (active && vi < nvec) {
        v[g0 + k] = load_pack<T, E, true>(xr + vi * E);
        if constexpr (RES) rv[k] = load_pack<T, E, true>(res + row * sr + vi * E);
      }
    }
    if constexpr (EW) {
      if (g0 == 0) {
#pragma unroll
        for (int k = 0; k < G; ++k) {
          const int vi = t + k * TPR;
          if (active && vi < nvec) wv[k].load(w + vi * E);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int vi = t + (g0 + k) * TPR;
      if (active && vi < nvec) {
        if constexpr (RES) {
#pragma unroll
          for (int e = 0; e < E; ++e)
            v[g0 + k].e[e] = from_f32<T>(to_f32(v[g0 + k].e[e]) + to_f32(rv[k].e[e]));
          if constexpr (WT)
            store_write_through<T, E>(rout + row * srout, hidden * static_cast<int>(sizeof(T)), vi * E, v[g0 + k]);
          else
            store_pack<T, E, true>(rout + row * srout + vi * E, v[g0 + k]);
        }
        ss = sumsq_add(v[g0 + k], ss);
      }
    }
  }
  // Elements past the last full packet (only when a row stride is padded).
  T vt = from_f32<T>(0.f);
  const int tcol = nvec * E + t;
  const bool has_tail = active && t < tail;
  if (has_tail) {
    vt = xr[tcol];
    if constexpr (RES) {
      vt = from_f32<T>(to_f32(vt) + to_f32(res[row * sr + tcol]));
      rout[row * srout + tcol] = vt;
    }
    const float f = to_f32(vt);
    ss = __builtin_fmaf(f, f, ss);
  }

  // The weight row is L2-resident (every row reads it); fetch the first group
  // before the reduction so its latency hides behind the cross-lane sums.
  if constexpr (kPrefetchW && !EW) {
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int vi = t + k * TPR;
      if (active && vi < nvec) wv[k].load(w + vi * E);
    }
  }

  ss = wave_sum(ss);
  if constexpr (WPR > 1) {
    __shared__ float partial[RPB][WPR];
    if (lane == 0) partial[row_in_block][wave_in_row] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int j = 0; j < WPR; ++j) ss += partial[row_in_block][j];
  }
  const float rstd = rsqrtf(ss * inv_h + eps);

#pragma unroll
  for (int g0 = 0; g0 < VPT; g0 += G) {
    if (g0 > 0 || !kPrefetchW) {
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int vi = t + (g0 + k) * TPR;
        if (active && vi < nvec) wv[k].load(w + vi * E);
      }
    }
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const int vi = t + (g0 + k) * TPR;
      if (active && vi < nvec) {
        P o;
#pragma unroll
        for (int e = 0; e < E; ++e) o.e[e] = from_f32<T>((to_f32(v[g0 + k].e[e]) * rstd) * wv[k][e]);
        if constexpr (WT)
          store_write_through<T, E>(yr, hidden * static_cast<int>(sizeof(T)), vi * E, o);
        else
          store_pack<T, E, true>(yr + vi * E, o);
      }
    }
  }
  if (has_tail) yr[tcol] = from_f32<T>((to_f32(vt) * rstd) * to_f32(w[tcol]));
}

// rmsnorm_pipe - rmsnorm_reg's row layout (WPR wavefronts per row, lane t
// holding packets t + k * 64 * WPR) in a persistent grid: a workgroup owns one
// row at a time and walks a sequence of rows, and it issues the loads of its
// next row before it reduces and writes the current one. In rmsnorm_reg a
// workgroup reads its row, waits, then only writes, so a CU's reads stall
// while its rows drain; here every wavefront keeps one row's reads in flight
// through its writes. The lane's slice of the weight row is the same for
// every row and is loaded once. Only full rows take this kernel
// (hidden = 64 * WPR * VPT * E), so every load is unconditional. The
// arithmetic and the order of every sum are rmsnorm_reg's, so the two
// kernels give bitwise-identical outputs.
//
// The loop holds two register buffers, A and B, and is unrolled by two with
// the first row peeled off, so that both ways into the loop head leave the
// same operations outstanding (B's loads, then one row's stores). The
// compiler's wait counts are then exact: consuming a buffer waits for that
// buffer's loads only, not for the stores issued after them (vmcnt counts
// loads and stores in one in-order queue on gfx950).
//
// Row sequence: with xcd_runs the rows are cut into 8 contiguous ranges, one
// per XCD (workgroup b runs on XCD b % 8; the grid is a multiple of 8), and
// the workgroups of one XCD interleave within its range; otherwise the grid
// strides over all rows.
template <typename T, int E, int VPT, int TPR, bool RES>
__device__ __forceinline__ void pipe_load(const T* __restrict__ xr, const T* __restrict__ rr, int t,
                                          Pack<T, E> (&vx)[VPT], Pack<T, E> (&vr)[VPT]) {
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    vx[k] = load_pack<T, E, true>(xr + (t + k * TPR) * E);
    if constexpr (RES) vr[k] = load_pack<T, E, true>(rr + (t + k * TPR) * E);
  }
}

template <typename T, typename W, int E, int VPT, int WPR, bool RES, int SLOT>
__device__ __forceinline__ void pipe_row(Pack<T, E> (&vx)[VPT], const Pack<T, E> (&vr)[VPT],
                                         const WeightPacket<W, E> (&wv)[VPT], float (&partial)[2][WPR],
                                         T* __restrict__ y, T* __restrict__ rout, int64_t row, int64_t sy,
                                         int64_t srout, int t, float inv_h, float eps) {
  constexpr int TPR = kWave * WPR;
  const int lane = t & (kWave - 1);
  const int wave = t / kWave;
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    if constexpr (RES) {
#pragma unroll
      for (int e = 0; e < E; ++e) vx[k].e[e] = from_f32<T>(to_f32(vx[k].e[e]) + to_f32(vr[k].e[e]));
      store_pack<T, E, true>(rout + row * srout + (t + k * TPR) * E, vx[k]);
    }
    ss = sumsq_add(vx[k], ss);
  }
  ss = wave_sum(ss);
  if constexpr (WPR > 1) {
    // Rows alternate between two slots: a wavefront one row ahead writes the
    // other slot, and cannot get two rows ahead without passing this barrier.
    if (lane == 0) partial[SLOT][wave] = ss;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    ss = 0.f;
#pragma unroll
    for (int j = 0; j < WPR; ++j) ss += partial[SLOT][j];
  }
  const float rstd = rsqrtf(ss * inv_h + eps);
#pragma unroll
  for (int k = 0; k < VPT; ++k) {
    Pack<T, E> o;
#pragma unroll
    for (int e = 0; e < E; ++e) o.e[e] = from_f32<T>((to_f32(vx[k].e[e]) * rstd) * wv[k][e]);
    store_pack<T, E, true>(y + row * sy + (t + k * TPR) * E, o);
  }
}

template <typename T, typename W, int WPR, int VPT, bool RES>
__global__ __launch_bounds__(kWave* WPR) void rmsnorm_pipe(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    T* __restrict__ y, T* __restrict__ rout, int64_t rows, int64_t sx, int64_t sr, int64_t sy,
    int64_t srout, float inv_h, float eps, int xcd_runs) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  constexpr int TPR = kWave * WPR;
  using P = Pack<T, E>;
  const int t = threadIdx.x;

  int64_t row, step, end;
  if (xcd_runs) {
    const int64_t xcd = blockIdx.x % 8, per_xcd = gridDim.x / 8;
    row = xcd * rows / 8 + blockIdx.x / 8;
    end = (xcd + 1) * rows / 8;
    step = per_xcd;
  } else {
    row = blockIdx.x;
    end = rows;
    step = gridDim.x;
  }
  if (row >= end) return;  // the whole workgroup: no barrier is reached
  // Rows of this workgroup: row + i * step for i < n (n < 2^31: the launcher
  // sends no more rows). The prefetch after the last row reads the weight
  // row instead (L2-resident, at least as long as one row of x, discarded),
  // so that every load is issued unconditionally.
  const int n = static_cast<int>((end - row + step - 1) / step);
  const T* spare = reinterpret_cast<const T*>(w);

  WeightPacket<W, E> wv[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) wv[k].load(w + (t + k * TPR) * E);
  __shared__ float partial[2][WPR];

  P ax[VPT], bx[VPT];
  [[maybe_unused]] P ar[VPT];
  [[maybe_unused]] P br[VPT];
  pipe_load<T, E, VPT, TPR, RES>(x + row * sx, res + row * sr, t, ax, ar);
  const bool two = n > 1;
  pipe_load<T, E, VPT, TPR, RES>(two ? x + (row + step) * sx : spare, two ? res + (row + step) * sr : spare, t, bx,
                                 br);
  pipe_row<T, W, E, VPT, WPR, RES, 0>(ax, ar, wv, partial, y, rout, row, sy, srout, t, inv_h, eps);
  int i = 1;
  for (; i + 1 < n; i += 2) {
    // Rows i (in B) and i + 1 exist; A takes row i + 1, then B row i + 2.
    const int64_t r = row + static_cast<int64_t>(i) * step;
    pipe_load<T, E, VPT, TPR, RES>(x + (r + step) * sx, res + (r + step) * sr, t, ax, ar);
    pipe_row<T, W, E, VPT, WPR, RES, 1>(bx, br, wv, partial, y, rout, r, sy, srout, t, inv_h, eps);
    const bool more = i + 2 < n;
    pipe_load<T, E, VPT, TPR, RES>(more ? x + (r + 2 * step) * sx : spare,
                                   more ? res + (r + 2 * step) * sr : spare, t, bx, br);
    pipe_row<T, W, E, VPT, WPR, RES, 0>(ax, ar, wv, partial, y, rout, r + step, sy, srout, t, inv_h, eps);
  }
  if (i < n)  // the last row, in B
    pipe_row<T, W, E, VPT, WPR, RES, 1>(bx, br, wv, partial, y, rout, row + static_cast<int64_t>(i) * step, sy,
                                        srout, t, inv_h, eps);
}

// Two-pass kernel: one workgroup of kStreamBlock lanes per row, packets of E
// elements (E = 16/sizeof(T) when aligned, else 1).
constexpr int kStreamBlock = 256;

template <typename T, typename W, int E, bool RES>
__global__ __launch_bounds__(kStreamBlock) void rmsnorm_stream(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    T* __restrict__ y, T* __restrict__ rout, int64_t row0, int hidden, int64_t sx, int64_t sr,
    int64_t sy, int64_t srout, float inv_h, float eps) {
  using P = Pack<T, E>;
  const int64_t row = row0 + blockIdx.x;
  const int tid = threadIdx.x;
  const int nvec = hidden / E;
  const int tail = hidden - nvec * E;
  const T* xr = x + row * sx;
  const T* rr = res + row * sr;  // only dereferenced when RES
  T* yr = y + row * sy;
  T* ror = rout + row * srout;

  // s = x (+ r rounded to T); the residual variant writes s in pass one and
  // recomputes it from the untouched inputs in pass two.
  auto element = [&](int col) -> T {
    if constexpr (RES) {
      return from_f32<T>(to_f32(xr[col]) + to_f32(rr[col]));
    } else {
      return xr[col];
    }
  };
  auto packet = [&](int vi) -> P {
    P p = load_pack<T, E>(xr + vi * E);
    if constexpr (RES) {
      const P q = load_pack<T, E>(rr + vi * E);
#pragma unroll
      for (int e = 0; e < E; ++e) p.e[e] = from_f32<T>(to_f32(p.e[e]) + to_f32(q.e[e]));
    }
    return p;
  };

  float ss = 0.f;
  for (int vi = tid; vi < nvec; vi += kStreamBlock) {
    const P p = packet(vi);
    if constexpr (RES) store_pack<T, E>(ror + vi * E, p);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float f = to_f32(p.e[e]);
      ss = __builtin_fmaf(f, f, ss);
    }
  }
  for (int j = tid; j < tail; j += kStreamBlock) {
    const T s = element(nvec * E + j);
    if constexpr (RES) ror[nvec * E + j] = s;
    const float f = to_f32(s);
    ss = __builtin_fmaf(f, f, ss);
  }

  ss = wave_sum(ss);
  __shared__ float partial[kStreamBlock / kWave];
  if ((tid & (kWave - 1)) == 0) partial[tid / kWave] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int j = 0; j < kStreamBlock / kWave; ++j) ss += partial[j];
  const float rstd = rsqrtf(ss * inv_h + eps);

  for (int vi = tid; vi < nvec; vi += kStreamBlock) {
    const P p = packet(vi);
    float wf[E];
    load_f32<W, E>(w + vi * E, wf);
    P o;
#pragma unroll
    for (int e = 0; e < E; ++e) o.e[e] = from_f32<T>((to_f32(p.e[e]) * rstd) * wf[e]);
    store_pack<T, E>(yr + vi * E, o);
  }
  for (int j = tid; j < tail; j += kStreamBlock) {
    const int col = nvec * E + j;
    yr[col] = from_f32<T>((to_f32(element(col)) * rstd) * to_f32(w[col]));
  }
}

// Tensor-parallel halves of (residual) RMSNorm, for a row whose hidden
// dimension is split over ranks. Each rank runs rmsnorm_shard_partial on its
// slice (s = x (+ r), rounded to T and written when there is a residual, and
// the fp32 sum of squares of s), the partial sums are all-reduced across the
// ranks, and rmsnorm_shard_apply normalises each slice with the total:
//   y = to_T((s * rsqrt(total * (1/H) + eps)) * w)
// with H the full hidden size, the same arithmetic as rmsnorm_reg. One
// 256-lane workgroup per row, packets of E elements (E = 1 when unaligned).
template <typename T, int E, bool RES>
__global__ __launch_bounds__(kStreamBlock) void rmsnorm_shard_partial(
    const T* __restrict__ x, const T* __restrict__ res, T* __restrict__ rout,
    float* __restrict__ partial, int64_t row0, int shard, int64_t sx, int64_t sr, int64_t srout) {
  using P = Pack<T, E>;
  const int64_t row = row0 + blockIdx.x;
  const int tid = threadIdx.x;
  const int nvec = shard / E;
  const T* xr = x + row * sx;
  float ss = 0.f;
  for (int vi = tid; vi < nvec; vi += kStreamBlock) {
    P p = load_pack<T, E, true>(xr + vi * E);
    if constexpr (RES) {
      const P q = load_pack<T, E, true>(res + row * sr + vi * E);
#pragma unroll
      for (int e = 0; e < E; ++e) p.e[e] = from_f32<T>(to_f32(p.e[e]) + to_f32(q.e[e]));
      store_pack<T, E, true>(rout + row * srout + vi * E, p);
    }
    ss = sumsq_add(p, ss);
  }
  for (int j = nvec * E + tid; j < shard; j += kStreamBlock) {  // tail (E > 1 only)
    T v = xr[j];
    if constexpr (RES) {
      v = from_f32<T>(to_f32(v) + to_f32(res[row * sr + j]));
      rout[row * srout + j] = v;
    }
    const float f = to_f32(v);
    ss = __builtin_fmaf(f, f, ss);
  }
  ss = wave_sum(ss);
  __shared__ float lds[kStreamBlock / kWave];
  if ((tid & (kWave - 1)) == 0) lds[tid / kWave] = ss;
  __syncthreads();
  if (tid == 0) {
    float total = 0.f;
#pragma unroll
    for (int j = 0; j < kStreamBlock / kWave; ++j) total += lds[j];
    partial[row] = total;
  }
}

template <typename T, typename W, int E, int R>
__global__ __launch_bounds__(kStreamBlock) void rmsnorm_shard_apply(
    const T* __restrict__ s, const W* __restrict__ w, const float* __restrict__ total,
    T* __restrict__ y, int64_t row0, int64_t rows, int shard, int64_t ss_, int64_t sy, float inv_h, float eps) {
  // Each workgroup applies R consecutive rows; a lane holds the same columns of
  // all R, so the weight packet is read once for R rows.
  using P = Pack<T, E>;
  const int64_t first = row0 + static_cast<int64_t>(blockIdx.x) * R;
  const int tid = threadIdx.x;
  const int nvec = shard / E;
  const auto apply = [&](int64_t row, int vi, const P& p, const float (&wf)[E], float rstd) {
    P o;
#pragma unroll
    for (int e = 0; e < E; ++e) o.e[e] = from_f32<T>((to_f32(p.e[e]) * rstd) * wf[e]);
    store_pack<T, E, true>(y + row * sy + vi * E, o);
  };
  // The data packets are requested before the rows' totals are read: a total
  // is a dependent read of its own (a scalar load), and computing rstd first
  // would put that round trip in front of every workgroup's data loads.
  float rstd[R];
  bool have_rstd = false;
  for (int vi = tid; vi < nvec; vi += kStreamBlock) {
    P p[R];
#pragma unroll
    for (int k = 0; k < R; ++k)
      if (first + k < rows) p[k] = load_pack<T, E, true>(s + (first + k) * ss_ + vi * E);
    float wf[E];
    load_f32<W, E>(w + vi * E, wf);
    if (!have_rstd) {
#pragma unroll
      for (int k = 0; k < R; ++k) rstd[k] = first + k < rows ? rsqrtf(total[first + k] * inv_h + eps) : 0.f;
      have_rstd = true;
    }
#pragma unroll
    for (int k = 0; k < R; ++k)
      if (first + k < rows) apply(first + k, vi, p[k], wf, rstd[k]);
  }
  const int tail0 = nvec * E + tid;
  if (tail0 < shard) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int64_t row = first + k;
      if (row >= rows) break;
      const float rs = rsqrtf(total[row] * inv_h + eps);
      const T* sr = s + row * ss_;
      T* yr = y + row * sy;
      for (int j = tail0; j < shard; j += kStreamBlock) yr[j] = from_f32<T>((to_f32(sr[j]) * rs) * to_f32(w[j]));
    }
  }
}

namespace {

// Launches of at most this many rows leave CUs without a workgroup (256 CUs).
constexpr int64_t kFewRows = 256;

struct RegShape {
  int wpr, vpt;
};
// Instantiated (waves per row, packets per lane) shapes, smallest first.
constexpr RegShape kRegShapes[] = {{1, 1}, {1, 2},  {1, 4},  {1, 8},  {2, 1},  {2, 2},  {2, 4},
                                   {2, 8}, {4, 1},  {4, 2},  {4, 4},  {4, 8},  {8, 1},  {8, 2},
                                   {8, 4}, {8, 8},  {16, 1}, {16, 2}, {16, 4}, {16, 8}};
// Widest row held in registers: 16 wavefronts x 64 lanes x 8 packets (65536
// half-precision elements). Wider rows take the two-pass kernel.
constexpr int kMaxRegPackets = 16 * 64 * 8;


// Default shape (waves per row, packets per lane). Medians of three cold runs
// per shape on MI355X, 16384 rows, fp16 and bf16: plain rows are fastest
// with two packets per lane over 4-16 wavefronts; residual rows, which load
// two tensors per packet, with one packet per lane over 8-16 wavefronts.
// Rows that fit one wavefront's first packet stay on one wavefront so that
// small rows need no LDS exchange and pack 4 rows per workgroup.
RegShape pick_shape(int64_t nvec, bool residual, int64_t rows) {
  // One packet per lane and more wavefronts per row for the residual variant,
  // and for plain rows when a launch has too few rows to give every CU a
  // workgroup (decode): then each row's latency is the launch's. Graph-replayed
  // on MI355X, plain rows of 4096 half elements take 1.89 us as (8, 1) against
  // 2.13 us as (4, 2) at 1 row (2.04 against 2.28 at 32 rows); at 16384 rows
  // (4, 2) is the faster.
  const bool one_packet = residual || rows <= kFewRows;
  RegShape s{16, 8};
  if (nvec <= 64) s = {1, 1};
  else if (nvec <= 128) s = {1, 2};
  else if (nvec <= 256) s = {2, 2};
  else if (nvec <= 512) s = one_packet ? RegShape{8, 1} : RegShape{4, 2};
  else if (nvec <= 1024) s = one_packet ? RegShape{16, 1} : RegShape{8, 2};
  else if (nvec <= 2048) s = {16, 2};
  else if (nvec <= 4096) s = {16, 4};
  const int want_wpr = g_rms_tuning.waves_per_row, want_vpt = g_rms_tuning.vecs_per_thread;
  if (want_wpr > 0 || want_vpt > 0) {
    RegShape want{want_wpr > 0 ? want_wpr : s.wpr, want_vpt > 0 ? want_vpt : s.vpt};
    for (const RegShape& c : kRegShapes)
      if (c.wpr == want.wpr && c.vpt == want.vpt && int64_t(c.wpr) * 64 * c.vpt >= nvec) return c;
  }
  return s;
}

constexpr unsigned kXcdChunk = 8;
// Residual rows of 16384 half elements (the one-workgroup-per-CU launches
// below, write-through stores, one packet per load group) take runs of 16.
// Medians of 7-10 rotating back-to-back runs on MI355X, same buffers, outputs
// identical, three boxes: runs of 16 gained 0.4-1.4 points of peak over runs
// of 8 (e.g. 81.5% / 82.7% against 80.3% / 81.3%, bf16 / fp16); runs of 12,
// 20, 24 and 32 were no better than 8, and the whole 12-launch step read
// 6542 against 6525 GB/s. Plain rows of 16384 and residual rows of 8192
// showed no consistent gain from 16. Runs of 4 read +0.1 to +0.3 over 16
// with random spacer allocations between the inputs (four placements on
// each of four boxes), but -0.9 (bf16) and -0.1 (fp16) with the inputs
// allocated back to back, five repetitions on each of two boxes, so 16
// stays.
constexpr unsigned kXcdChunkWideResidual = 16;
// Plain rows of 16384 half elements take runs of 4. Five buffer placements
// (random spacer allocations between the input copies) on each of three
// MI355X boxes, variants interleaved, medians of settled back-to-back runs:
// against runs of 8, fp16 +0.29 to +0.30 points of peak (per-placement
// -0.06 to +0.71), bf16 +0.56 to +0.70 (+0.20 to +0.97); runs of 16 were
// -0.23 to -0.29. With the inputs allocated back to back: bf16 +0.7 to
// +0.9 over runs of 8 on two boxes.
constexpr unsigned kXcdChunkWidePlain = 4;

// Workgroups per launch: at most 2^31 work-items, so the 32-bit grid size of
// the dispatch packet never wraps; larger problems take several launches,
// each starting at row0. ako_set_tuning(0, 7, n) lowers the cap (tests
// exercise the split at small sizes with it).
int64_t max_blocks_per_launch(int threads_per_block) {
  const int64_t cap = (int64_t(1) << 31) / threads_per_block;
  const int64_t forced = g_rms_tuning.max_blocks;
  return forced > 0 ? std::min(cap, forced) : cap;
}

template <typename T, typename W, int WPR, int VPT, bool RES, bool EW, bool SPLIT = false, bool WT = false>
hipError_t run_reg_launch(const RmsArgs& a, hipStream_t stream) {
  constexpr int RPB = WPR >= 4 ? 1 : 4 / WPR;
  const dim3 block(kWave * WPR * RPB);
  const int64_t total_blocks = ceil_div(a.rows, RPB);
  const int64_t cap = max_blocks_per_launch(kWave * WPR * RPB);
  // A residual row of >= 32 KiB per tensor keeps 4 x 32 KiB in flight; two
  // such rows per CU exceed the CU's share of its XCD's L2 (4 MiB / 32 CUs),
  // so an LDS reservation above half the CU's 160 KiB limits those launches to
  // one 16-wavefront workgroup per CU (measured +1-3% at 16384 x 16384).
  const bool row32k = a.hidden * static_cast<int64_t>(sizeof(T)) >= 32 * 1024;
  const bool one_per_cu = RES && WPR == 16 && row32k;
  unsigned lds = static_cast<unsigned>(g_rms_tuning.lds_reserve);
  if (lds == 0 && one_per_cu) lds = 82 * 1024;
  unsigned run = kXcdChunk;
  if (WPR == 16 && VPT == 2 && sizeof(T) == 2 && row32k) run = RES ? kXcdChunkWideResidual : kXcdChunkWidePlain;
  // Default: rows of >= 16 KiB go to the XCDs in runs of 8 consecutive rows
  // (rows of 16384 half elements: 16 residual, 4 plain; once the launch
  // holds 8 such runs); narrower rows keep block order.
  // Medians of 5 cold runs on MI355X, 16384 rows, fp16/bf16, against block
  // order: +1% at 16 KiB rows, +4% (plain) and +8-10% (residual) at 32 KiB
  // rows, -1-2% at 8 KiB rows; whole-grid runs (chunk = n / 8) lose up to 12%
  // at 8 KiB rows.
  const bool wide = a.hidden * static_cast<int64_t>(sizeof(T)) >= 16 * 1024;
  for (int64_t b0 = 0; b0 < total_blocks; b0 += cap) {
    const dim3 grid(static_cast<unsigned>(std::min(cap, total_blocks - b0)));
    unsigned xcd_chunk = !wide ? 1u : grid.x >= 8 * run ? run : grid.x >= 8 * kXcdChunk ? kXcdChunk : 1u;
    const int order = g_rms_tuning.row_order, chunk = g_rms_tuning.xcd_chunk;
    if (order == 1) xcd_chunk = 1;
    if (order == 2) xcd_chunk = chunk > 0 ? unsigned(chunk) : unsigned(grid.x / 8);
    AKO_LAUNCH((rmsnorm_reg<T, W, WPR, VPT, RPB, RES, EW, SPLIT, WT>),
               grid, block, lds, stream, static_cast<const T*>(a.x), static_cast<const T*>(a.r),
               static_cast<const W*>(a.w), static_cast<T*>(a.y), static_cast<T*>(a.rout),
               b0 * RPB, a.rows, static_cast<int>(a.hidden), a.sx, a.sr, a.sy, a.srout,
               1.0f / static_cast<float>(a.hidden), a.eps, make_xcd_runs(xcd_chunk));
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

// Early weight loads (EW) for launches of at most kFewRows rows of at most
// 8 KiB, whose time is one row's dependent chain. Graph-replayed on MI355X
// with inputs evicted from every cache (64 calls on separate inputs after an
// eviction pass), rows of 4096 half elements: residual 2.89 -> 2.64 us (1 row)
// and 3.09 -> 2.94 us (32 rows), plain 2.50 -> 2.43 us; with hot inputs the
// plain row gains 4% and the residual row loses 4%. Rows of 8192 and 16384
// elements are 2-13% slower with early weights, hot and cold (more requests
// per lane ahead of the reduction), so they keep the late loads, as do
// launches of many rows, whose weight row is L2-resident after the first rows.
// Only the one- and two-packet shapes (what decode rows use) have the variant.
constexpr int64_t kEarlyWeightRowBytes = 8 * 1024;

template <typename T, typename W, int WPR, int VPT, bool RES>
hipError_t run_reg(const RmsArgs& a, hipStream_t stream) {
  if constexpr (VPT <= 2) {
    const int forced = g_rms_tuning.early_weights;
    const bool ew = forced == 2 ||
                    (forced == 0 && a.rows <= kFewRows &&
                     a.hidden * static_cast<int64_t>(sizeof(T)) <= kEarlyWeightRowBytes);
    if (ew) return run_reg_launch<T, W, WPR, VPT, RES, true>(a, stream);
  }
  // Without write-through stores (key 12 = 1): one packet per load group for
  // bf16 residual rows of 16 wavefronts x 2 packets in launches of many rows.
  // Medians of 10 interleaved repetitions on MI355X, 16384 x 16384, cold
  // inputs, non-temporal stores: bf16 +1.5% back to back and +1.9% per launch;
  // fp16 -0.3%, so fp16 keeps whole groups, as do plain rows (-1.4% bf16,
  // -3.5% fp16).
  // Rows of 8193-16384 elements at 16 wavefronts x 2 packets in launches of
  // many rows store write-through (see store_write_through); residual rows
  // then take one packet per load group, fp16 and bf16 alike. fp32 rows of
  // 8192 on the same shape: plain 80.6% against 78.2% with non-temporal
  // stores, residual 82.5% against 81.2%. Rows at 16 wavefronts x 1 packet
  // (4097-8192 elements) keep non-temporal stores by default: residual rows
  // of 8192, five buffer placements on each of three MI355X boxes, variants
  // interleaved, write-through was -0.43 to -0.55 points of peak for bf16
  // (every placement -0.17 or worse) and -0.33 to -0.42 for fp16. Key 12 = 2
  // still selects it there.
  if constexpr ((VPT == 2 || VPT == 1) && WPR == 16) {
    constexpr bool kWtByDefault = VPT == 2;
    const int wt_forced = g_rms_tuning.write_through;
    if (wt_forced == 2 || (wt_forced == 0 && kWtByDefault && a.rows > kFewRows)) {
      if constexpr (RES) {
        if (g_rms_tuning.load_groups != 1) return run_reg_launch<T, W, WPR, VPT, RES, false, true, true>(a, stream);
      }
      return run_reg_launch<T, W, WPR, VPT, RES, false, false, true>(a, stream);
    }
  }
  if constexpr (VPT == 2 && WPR == 16 && RES) {
    const int forced = g_rms_tuning.load_groups;
    const bool split = forced == 2 || (forced == 0 && std::is_same_v<T, __bf16> && a.rows > kFewRows);
    if (split) return run_reg_launch<T, W, WPR, VPT, RES, false, true>(a, stream);
  }
  return run_reg_launch<T, W, WPR, VPT, RES, false>(a, stream);
}

// Compute units of the current device (the pipelined grid's size), read
// once per device.
int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Widest input row (x, plus the residual) the pipelined kernel takes by
// default, and the fewest rows per workgroup at which plain rows take it.
constexpr int64_t kPipeMaxRowBytes = 16 * 1024;
constexpr int64_t kPipeMinRowsPerBlock = 16;

// Shapes with a pipelined instantiation (the defaults of launches of many
// rows up to 65536 half-precision elements, and their neighbours).
constexpr RegShape kPipeShapes[] = {{4, 2}, {8, 1}, {8, 2}, {16, 1}, {16, 2}, {16, 4}};

bool pipe_shape(const RegShape& s) {
  for (const RegShape& c : kPipeShapes)
    if (c.wpr == s.wpr && c.vpt == s.vpt) return true;
  return false;
}

// Workgroups of a pipelined launch (a multiple of 8). Workgroups per CU: 16
// wavefronts per CU for plain rows, 8 for residual rows (two tensors in
// flight per row). Measured at 16384 rows of 4096 half elements: plain 6598
// GB/s with 16 wavefronts per CU against 6029 with 8; residual 6976 with 8
// against 6826 with 16.
int64_t pipe_blocks(int wpr, bool residual, int64_t rows) {
  const int forced = g_rms_tuning.pipe_blocks_per_cu;
  const int64_t per_cu = forced > 0 ? forced : std::max(1, (residual ? 8 : 16) / wpr);
  const int64_t blocks = std::min<int64_t>(rows, per_cu * device_cus());
  return std::max<int64_t>(8, blocks / 8 * 8);
}

template <typename T, typename W, int WPR, int VPT, bool RES>
hipError_t run_pipe(const RmsArgs& a, hipStream_t stream) {
  const int64_t blocks = pipe_blocks(WPR, RES, a.rows);
  const int xcd_runs = g_rms_tuning.row_order == 1 ? 0 : 1;
  AKO_LAUNCH((rmsnorm_pipe<T, W, WPR, VPT, RES>), dim3(static_cast<unsigned>(blocks)), dim3(kWave * WPR),
             0, stream, static_cast<const T*>(a.x), static_cast<const T*>(a.r),
             static_cast<const W*>(a.w), static_cast<T*>(a.y), static_cast<T*>(a.rout), a.rows, a.sx,
             a.sr, a.sy, a.srout, 1.0f / static_cast<float>(a.hidden), a.eps, xcd_runs);
  return hipGetLastError();
}

template <typename T, typename W, bool RES>
hipError_t run_pipe_shape(const RegShape& s, const RmsArgs& a, hipStream_t stream) {
#define AKO_PIPE_SHAPE(WPR, VPT) \
  if (s.wpr == WPR && s.vpt == VPT) return run_pipe<T, W, WPR, VPT, RES>(a, stream);
  AKO_PIPE_SHAPE(4, 2)
  AKO_PIPE_SHAPE(8, 1)
  AKO_PIPE_SHAPE(8, 2)
  AKO_PIPE_SHAPE(16, 1)
  AKO_PIPE_SHAPE(16, 2)
  AKO_PIPE_SHAPE(16, 4)
#undef AKO_PIPE_SHAPE
  return hipErrorInvalidValue;
}

template <typename T, typename W, bool RES>
hipError_t run_reg_shape(const RegShape& s, const RmsArgs& a, hipStream_t stream) {
#define AKO_RMS_SHAPE(WPR, VPT) \
  if (s.wpr == WPR && s.vpt == VPT) return run_reg<T, W, WPR, VPT, RES>(a, stream);
  AKO_RMS_SHAPE(1, 1)
  AKO_RMS_SHAPE(1, 2)
  AKO_RMS_SHAPE(1, 4)
  AKO_RMS_SHAPE(1, 8)
  AKO_RMS_SHAPE(2, 1)
  AKO_RMS_SHAPE(2, 2)
  AKO_RMS_SHAPE(2, 4)
  AKO_RMS_SHAPE(2, 8)
  AKO_RMS_SHAPE(4, 1)
  AKO_RMS_SHAPE(4, 2)
  AKO_RMS_SHAPE(4, 4)
  AKO_RMS_SHAPE(4, 8)
  AKO_RMS_SHAPE(8, 1)
  AKO_RMS_SHAPE(8, 2)
  AKO_RMS_SHAPE(8, 4)
  AKO_RMS_SHAPE(8, 8)
  AKO_RMS_SHAPE(16, 1)
  AKO_RMS_SHAPE(16, 2)
  AKO_RMS_SHAPE(16, 4)
  AKO_RMS_SHAPE(16, 8)
#undef AKO_RMS_SHAPE
  return hipErrorInvalidValue;
}

template <typename T, typename W, bool RES>
hipError_t run_stream(const RmsArgs& a, hipStream_t stream) {
  const float inv_h = 1.0f / static_cast<float>(a.hidden);
  const auto* x = static_cast<const T*>(a.x);
  const auto* r = static_cast<const T*>(a.r);
  const auto* w = static_cast<const W*>(a.w);
  auto* y = static_cast<T*>(a.y);
  auto* ro = static_cast<T*>(a.rout);
  const int h = static_cast<int>(a.hidden);
  const int64_t cap = max_blocks_per_launch(kStreamBlock);
  for (int64_t r0 = 0; r0 < a.rows; r0 += cap) {
    const dim3 grid(static_cast<unsigned>(std::min(cap, a.rows - r0)));
    if (a.vector_ok) {
      AKO_LAUNCH((rmsnorm_stream<T, W, 16 / sizeof(T), RES>), grid, dim3(kStreamBlock), 0,
                 stream, x, r, w, y, ro, r0, h, a.sx, a.sr, a.sy, a.srout, inv_h, a.eps);
    } else {
      AKO_LAUNCH((rmsnorm_stream<T, W, 1, RES>), grid, dim3(kStreamBlock), 0, stream, x, r,
                 w, y, ro, r0, h, a.sx, a.sr, a.sy, a.srout, inv_h, a.eps);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

template <typename T, typename W>
hipError_t run_typed(const RmsArgs& a, hipStream_t stream) {
  constexpr int E = 16 / sizeof(T);
  const int64_t nvec = a.hidden / E;
  const bool reg = a.vector_ok && g_rms_tuning.force_stream == 0 && nvec <= kMaxRegPackets &&
                   nvec >= 1;
  if (!reg) return a.residual ? run_stream<T, W, true>(a, stream) : run_stream<T, W, false>(a, stream);
  RegShape s = pick_shape(nvec, a.residual, a.rows);
  // The pipelined kernel takes full rows only (no packet past the row's end)
  // and launches of many rows. By default it runs rows of 512 or 1024
  // packets whose inputs (x, and the residual) total at most 16 KiB, as one
  // packet per lane per tensor over nvec / 64 wavefronts. Medians of five
  // cold back-to-back runs on MI355X, 16384 rows, against rmsnorm_reg's
  // default: plain rows of 4096 half elements 5947 -> 6568 GB/s, residual
  // rows of 4096 6143 -> 6978, plain rows of 8192 6340 -> 7001, fp32 rows of
  // 2048 and 4096 +10-15% alike. Rows of 32 KiB of input (residual 8192,
  // plain and residual 16384), and two packets per lane at any width, were
  // 3-18% slower pipelined. Plain rows need 16 rows per workgroup: with 2-4
  // (512 or 2048 rows) they ran 7-15% slower than rmsnorm_reg, while
  // residual rows were as fast or faster from 300 rows up.
  const bool rows_ok = a.rows > kFewRows && a.rows < (int64_t(1) << 31) && nvec * E == a.hidden;
  const bool forced_shape = g_rms_tuning.waves_per_row > 0 || g_rms_tuning.vecs_per_thread > 0;
  bool pipe = false;
  if (g_rms_tuning.pipeline == 2) {
    pipe = rows_ok && int64_t(s.wpr) * kWave * s.vpt == nvec && pipe_shape(s);
  } else if (g_rms_tuning.pipeline == 0 && !forced_shape && rows_ok && (nvec == 512 || nvec == 1024) &&
             a.hidden * static_cast<int64_t>(sizeof(T)) * (a.residual ? 2 : 1) <= kPipeMaxRowBytes) {
    const RegShape one{static_cast<int>(nvec / kWave), 1};
    if (a.residual || a.rows >= kPipeMinRowsPerBlock * pipe_blocks(one.wpr, false, a.rows)) {
      s = one;
      pipe = true;
    }
  }
  if (pipe) return a.residual ? run_pipe_shape<T, W, true>(s, a, stream) : run_pipe_shape<T, W, false>(s, a, stream);
  return a.residual ? run_reg_shape<T, W, true>(s, a, stream)
                    : run_reg_shape<T, W, false>(s, a, stream);
}

}  // namespace

namespace {

template <typename T, bool RES>
hipError_t run_shard_partial(const RmsShardArgs& a, hipStream_t stream) {
  const int64_t cap = max_blocks_per_launch(kStreamBlock);
  for (int64_t r0 = 0; r0 < a.rows; r0 += cap) {
    const dim3 grid(static_cast<unsigned>(std::min(cap, a.rows - r0)));
    if (a.vector_ok) {
      AKO_LAUNCH((rmsnorm_shard_partial<T, 16 / sizeof(T), RES>), grid, dim3(kStreamBlock), 0,
                 stream, static_cast<const T*>(a.x), static_cast<const T*>(a.r),
                 static_cast<T*>(a.rout), a.partial, r0, static_cast<int>(a.shard), a.sx,
                 a.sr, a.srout);
    } else {
      AKO_LAUNCH((rmsnorm_shard_partial<T, 1, RES>), grid, dim3(kStreamBlock), 0, stream,
                 static_cast<const T*>(a.x), static_cast<const T*>(a.r),
                 static_cast<T*>(a.rout), a.partial, r0, static_cast<int>(a.shard), a.sx,
                 a.sr, a.srout);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

template <typename T, typename W, int R>
hipError_t run_shard_apply_r(const RmsShardArgs& a, hipStream_t stream) {
  const int64_t cap = max_blocks_per_launch(kStreamBlock) * R;  // rows per launch
  const float inv_h = 1.0f / static_cast<float>(a.hidden);
  for (int64_t r0 = 0; r0 < a.rows; r0 += cap) {
    const int64_t end = std::min(a.rows, r0 + cap);
    const dim3 grid(static_cast<unsigned>(ceil_div(end - r0, R)));
    if (a.vector_ok) {
      AKO_LAUNCH((rmsnorm_shard_apply<T, W, 16 / sizeof(T), R>), grid, dim3(kStreamBlock), 0,
                 stream, static_cast<const T*>(a.x), static_cast<const W*>(a.w), a.total,
                 static_cast<T*>(a.y), r0, end, static_cast<int>(a.shard), a.sx, a.sy, inv_h,
                 a.eps);
    } else {
      AKO_LAUNCH((rmsnorm_shard_apply<T, W, 1, R>), grid, dim3(kStreamBlock), 0, stream,
                 static_cast<const T*>(a.x), static_cast<const W*>(a.w), a.total,
                 static_cast<T*>(a.y), r0, end, static_cast<int>(a.shard), a.sx, a.sy, inv_h,
                 a.eps);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

// Rows per workgroup: 2 for launches with enough rows to fill the chip many
// times over, 1 for decode-sized ones (which need every workgroup they can
// get). On MI355X, 16384 rows of a 2048-element slice: two rows per workgroup
// beat one, and four were no faster than two.
template <typename T, typename W>
hipError_t run_shard_apply(const RmsShardArgs& a, hipStream_t stream) {
  if (a.rows >= 4096) return run_shard_apply_r<T, W, 2>(a, stream);
  return run_shard_apply_r<T, W, 1>(a, stream);
}

}  // namespace

hipError_t launch_rmsnorm_shard_partial(const RmsShardArgs& a, hipStream_t stream) {
  switch (a.dtype) {
    case kF32: return a.residual ? run_shard_partial<float, true>(a, stream) : run_shard_partial<float, false>(a, stream);
    case kF16: return a.residual ? run_shard_partial<_Float16, true>(a, stream) : run_shard_partial<_Float16, false>(a, stream);
    case kBF16: return a.residual ? run_shard_partial<__bf16, true>(a, stream) : run_shard_partial<__bf16, false>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rmsnorm_shard_apply(const RmsShardArgs& a, hipStream_t stream) {
  const bool w_same = a.w_dtype == a.dtype;
  switch (a.dtype) {
    case kF32: return run_shard_apply<float, float>(a, stream);
    case kF16: return w_same ? run_shard_apply<_Float16, _Float16>(a, stream) : run_shard_apply<_Float16, float>(a, stream);
    case kBF16: return w_same ? run_shard_apply<__bf16, __bf16>(a, stream) : run_shard_apply<__bf16, float>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rmsnorm(const RmsArgs& a, hipStream_t stream) {
  const bool w_same = a.w_dtype == a.dtype;
  switch (a.dtype) {
    case kF32:
      return run_typed<float, float>(a, stream);
    case kF16:
      return w_same ? run_typed<_Float16, _Float16>(a, stream) : run_typed<_Float16, float>(a, stream);
    case kBF16:
      return w_same ? run_typed<__bf16, __bf16>(a, stream) : run_typed<__bf16, float>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace ako

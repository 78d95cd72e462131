// RMSNorm and residual-add + RMSNorm for gfx950.
//
// Two kernels:
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

#include "common.h"
#include "launch.h"

#ifndef AKO_RMS_PREFETCH_W
#define AKO_RMS_PREFETCH_W 1
#endif

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

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on
// XCD b % 8). block_order hands each XCD runs of `chunk` consecutive blocks:
// workgroup b = 8 i + x takes block c * 8 chunk + x * chunk + j for
// i = c * chunk + j, so the XCDs walk 8 separate runs instead of interleaving
// block by block. chunk <= 1 is the identity; the last, partial round of runs
// is split evenly the same way and the n % 8 trailing blocks keep their own
// index, which keeps the map a bijection on [0, n).
__device__ __forceinline__ unsigned block_order(unsigned b, unsigned n, unsigned chunk) {
  const unsigned q = n / 8;
  if (chunk <= 1 || b >= 8 * q) return b;
  const unsigned x = b % 8, i = b / 8;
  const unsigned full = q / chunk;
  const unsigned c = i / chunk, j = i % chunk;
  if (c < full) return c * 8 * chunk + x * chunk + j;
  const unsigned rest = q - full * chunk;
  return full * 8 * chunk + x * rest + (i - full * chunk);
}

template <typename T, typename W, int WPR, int VPT, int RPB, bool RES, bool NTL, bool NTS, bool EW>
__global__ __launch_bounds__(kWave* WPR* RPB) void rmsnorm_reg(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    T* __restrict__ y, T* __restrict__ rout, int64_t row0, int64_t rows, int hidden, int64_t sx,
    int64_t sr, int64_t sy, int64_t srout, float inv_h, float eps, unsigned xcd_chunk) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements per packet
  constexpr int TPR = kWave * WPR;                     // lanes per row
  // Packets are processed in groups: every load of a group is issued before
  // the first of them is consumed, so a lane's memory latency is paid once
  // per group rather than once per packet. Groups stay small enough that x,
  // the residual and the prefetched weights fit in registers.
  constexpr int G = VPT <= 4 ? VPT : (VPT <= 8 ? 4 : 2);
  static_assert(VPT % G == 0, "VPT must be a multiple of the group size");
  // With few packets per lane the first weight group is fetched before the
  // reduction; with many, registers are kept for x and weights come per group.
  // EW (early weights, decode-sized launches) issues the first weight group in
  // the same batch as the row's own loads: a launch of a few rows is one
  // dependent chain, and a norm weight that the rest of a model step has
  // evicted then costs one HBM round trip instead of a second one after x.
  static_assert(!EW || VPT <= 4, "early weights need the first group's weights in registers");
  constexpr bool kPrefetchW = (AKO_RMS_PREFETCH_W != 0 || EW) && VPT <= 4;
  using P = Pack<T, E>;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row_in_block = wave / WPR;
  const int wave_in_row = wave - row_in_block * WPR;
  const int t = wave_in_row * kWave + lane;
  const int64_t row = row0 + static_cast<int64_t>(block_order(blockIdx.x, gridDim.x, xcd_chunk)) * RPB + row_in_block;
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
        v[g0 + k] = load_pack<T, E, NTL>(xr + vi * E);
        if constexpr (RES) rv[k] = load_pack<T, E, NTL>(res + row * sr + vi * E);
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
          store_pack<T, E, NTS>(rout + row * srout + vi * E, v[g0 + k]);
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
        store_pack<T, E, NTS>(yr + vi * E, o);
      }
    }
  }
  if (has_tail) yr[tcol] = from_f32<T>((to_f32(vt) * rstd) * to_f32(w[tcol]));
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

#ifndef AKO_RMS_NT
#define AKO_RMS_NT 1
#endif
#ifndef AKO_RMS_NT_STORE
#define AKO_RMS_NT_STORE AKO_RMS_NT
#endif

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
  const RmsTuning& tu = g_rms_tuning;
  if (tu.waves_per_row > 0 || tu.vecs_per_thread > 0) {
    RegShape want{tu.waves_per_row > 0 ? tu.waves_per_row : s.wpr,
                  tu.vecs_per_thread > 0 ? tu.vecs_per_thread : s.vpt};
    for (const RegShape& c : kRegShapes)
      if (c.wpr == want.wpr && c.vpt == want.vpt && int64_t(c.wpr) * 64 * c.vpt >= nvec) return c;
  }
  return s;
}

constexpr unsigned kXcdChunk = 8;

// Workgroups per launch: at most 2^31 work-items, so the 32-bit grid size of
// the dispatch packet never wraps; larger problems take several launches,
// each starting at row0. ako_set_tuning(0, 7, n) lowers the cap (tests
// exercise the split at small sizes with it).
int64_t max_blocks_per_launch(int threads_per_block) {
  const int64_t cap = (int64_t(1) << 31) / threads_per_block;
  const int64_t forced = g_rms_tuning.max_blocks;
  return forced > 0 ? std::min(cap, forced) : cap;
}

template <typename T, typename W, int WPR, int VPT, bool RES, bool EW>
hipError_t run_reg_launch(const RmsArgs& a, hipStream_t stream) {
  constexpr int RPB = WPR >= 4 ? 1 : 4 / WPR;
  const dim3 block(kWave * WPR * RPB);
  const int64_t total_blocks = ceil_div(a.rows, RPB);
  const int64_t cap = max_blocks_per_launch(kWave * WPR * RPB);
  // A residual row of >= 32 KiB per tensor keeps 4 x 32 KiB in flight; two
  // such rows per CU exceed the CU's share of its XCD's L2 (4 MiB / 32 CUs),
  // so an LDS reservation above half the CU's 160 KiB limits those launches to
  // one 16-wavefront workgroup per CU (measured +1-3% at 16384 x 16384).
  unsigned lds = static_cast<unsigned>(g_rms_tuning.lds_reserve);
  if (lds == 0 && RES && WPR == 16 && a.hidden * static_cast<int64_t>(sizeof(T)) >= 32 * 1024)
    lds = 82 * 1024;
  // Default: rows of >= 16 KiB go to the XCDs in runs of 8 consecutive rows
  // (once the launch holds 8 such runs); narrower rows keep block order.
  // Medians of 5 cold runs on MI355X, 16384 rows, fp16/bf16, against block
  // order: +1% at 16 KiB rows, +4% (plain) and +8-10% (residual) at 32 KiB
  // rows, -1-2% at 8 KiB rows; whole-grid runs (chunk = n / 8) lose up to 12%
  // at 8 KiB rows.
  const bool wide = a.hidden * static_cast<int64_t>(sizeof(T)) >= 16 * 1024;
  for (int64_t b0 = 0; b0 < total_blocks; b0 += cap) {
    const dim3 grid(static_cast<unsigned>(std::min(cap, total_blocks - b0)));
    unsigned xcd_chunk = wide && grid.x >= 8 * kXcdChunk ? kXcdChunk : 1;
    if (g_rms_tuning.row_order == 1) xcd_chunk = 1;
    if (g_rms_tuning.row_order == 2)
      xcd_chunk = g_rms_tuning.xcd_chunk > 0 ? unsigned(g_rms_tuning.xcd_chunk) : unsigned(grid.x / 8);
    hipLaunchKernelGGL((rmsnorm_reg<T, W, WPR, VPT, RPB, RES, AKO_RMS_NT != 0, AKO_RMS_NT_STORE != 0, EW>), grid,
                       block, lds, stream, static_cast<const T*>(a.x), static_cast<const T*>(a.r),
                       static_cast<const W*>(a.w), static_cast<T*>(a.y), static_cast<T*>(a.rout),
                       b0 * RPB, a.rows, static_cast<int>(a.hidden), a.sx, a.sr, a.sy, a.srout,
                       1.0f / static_cast<float>(a.hidden), a.eps, xcd_chunk);
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
  return run_reg_launch<T, W, WPR, VPT, RES, false>(a, stream);
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
      hipLaunchKernelGGL((rmsnorm_stream<T, W, 16 / sizeof(T), RES>), grid, dim3(kStreamBlock), 0,
                         stream, x, r, w, y, ro, r0, h, a.sx, a.sr, a.sy, a.srout, inv_h, a.eps);
    } else {
      hipLaunchKernelGGL((rmsnorm_stream<T, W, 1, RES>), grid, dim3(kStreamBlock), 0, stream, x, r,
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
  const RegShape s = pick_shape(nvec, a.residual, a.rows);
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
      hipLaunchKernelGGL((rmsnorm_shard_partial<T, 16 / sizeof(T), RES>), grid, dim3(kStreamBlock), 0,
                         stream, static_cast<const T*>(a.x), static_cast<const T*>(a.r),
                         static_cast<T*>(a.rout), a.partial, r0, static_cast<int>(a.shard), a.sx,
                         a.sr, a.srout);
    } else {
      hipLaunchKernelGGL((rmsnorm_shard_partial<T, 1, RES>), grid, dim3(kStreamBlock), 0, stream,
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
      hipLaunchKernelGGL((rmsnorm_shard_apply<T, W, 16 / sizeof(T), R>), grid, dim3(kStreamBlock), 0,
                         stream, static_cast<const T*>(a.x), static_cast<const W*>(a.w), a.total,
                         static_cast<T*>(a.y), r0, end, static_cast<int>(a.shard), a.sx, a.sy, inv_h,
                         a.eps);
    } else {
      hipLaunchKernelGGL((rmsnorm_shard_apply<T, W, 1, R>), grid, dim3(kStreamBlock), 0, stream,
                         static_cast<const T*>(a.x), static_cast<const W*>(a.w), a.total,
                         static_cast<T*>(a.y), r0, end, static_cast<int>(a.shard), a.sx, a.sy, inv_h,
                         a.eps);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

#ifndef AKO_TP_APPLY_ROWS
#define AKO_TP_APPLY_ROWS 2
#endif

// Rows per workgroup: R for launches with enough rows to fill the chip many
// times over, 1 for decode-sized ones (which need every workgroup they can get).
template <typename T, typename W>
hipError_t run_shard_apply(const RmsShardArgs& a, hipStream_t stream) {
  if (AKO_TP_APPLY_ROWS >= 4 && a.rows >= 4096) return run_shard_apply_r<T, W, 4>(a, stream);
  if (AKO_TP_APPLY_ROWS >= 2 && a.rows >= 4096) return run_shard_apply_r<T, W, 2>(a, stream);
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

// Rotary position embedding (neox and interleaved pairing) for gfx950.
//
// rope_vec - one wavefront per token (b, s). The 64 lanes of the wavefront
//   are laid out as [heads in flight][packets per unit]:
//     neox:        a unit is one half of a head; lane j loads packet j of the
//                  lower half and packet j of the upper half (the pair
//                  partners sit exactly head_dim/2 apart);
//     interleaved: a unit is a whole head; each 16-byte packet holds E/2
//                  complete (2i, 2i+1) pairs.
//   A lane loads its slice of the cos/sin row once and reuses it for every
//   head it rotates, so the tables cost one L2 read per token instead of one
//   per head. ITERS head groups are loaded before any is computed, giving
//   each lane up to 2*ITERS independent 16-byte loads in flight. Both tensors
//   of a (q, k) pair can be rotated by the same wavefront (heads of the second
//   tensor continue the head index), which is how ako_rope_qk_fwd runs in one
//   launch.
//
// rope_scalar - any head_dim, any alignment: one lane per rotated pair.
//
// Both kernels have a KV-cache mode (CACHE): the position of token s is read
// on the device (*pos + s), the tables are read at that row, q is rotated to
// its output, k is rotated into slot *pos + s of the key cache and v is copied
// into the same slot of the value cache, all in the one launch. A captured
// decode step can then be replayed while *pos advances.
//
// Numerics follow ako/ops/rope_ref.py:73-107: a' = a*c - b*n and
// b' = a*n + b*c in fp32 with each product rounded separately (the library is
// built with -ffp-contract=off), then rounded to the storage dtype.

#include <algorithm>

#include "common.h"
#include "launch.h"

namespace ako {

RopeTuning g_rope_tuning;

struct RopeTensorDev {
  const void* x;
  void* y;
  int64_t heads;
  int64_t sxb, sxs, sxh;
  int64_t syb, sys, syh;
};

struct RopeDev {
  RopeTensorDev t0, t1, t2;  // t2: copied, not rotated (KV-cache mode only)
  const int64_t* pos;        // KV-cache mode: device-side position of token s = 0
  int64_t cache_len;
  const void* cos;
  const void* sin;
  int token0;        // first token of this launch (launches split at token boundaries)
  int tokens;        // tokens in this launch
  int chunks;        // head chunks (wavefronts) per token
  int seq;
  int head_dim;
  int pu_shift;      // log2(packets per unit) when a power of two, else -1
  int64_t st;
  int64_t total_tokens;  // batch * seq (scalar kernel)
  FastDiv by_chunks, by_seq;  // dividers for chunks and seq (vector kernel)
  XcdRuns runs;               // workgroup order over the XCDs (vector kernel)
};

template <typename T, typename TT, bool NEOX, int ITERS, int TPB, bool CACHE>
__global__ __launch_bounds__(kWave* TPB) void rope_vec(RopeDev a) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  constexpr int NT = NEOX ? E : E / 2;  // table values per lane
  using P = Pack<T, E>;

  // Wavefront w of this launch rotates head chunk (w % chunks) of token
  // token0 + w / chunks. All index arithmetic is 32-bit (the host splits
  // launches so that w < 2^24 and validates batch * seq < 2^31).
  // Spare wavefronts of the last workgroup and lanes past the last head group
  // are not sent away early: they compute clamped, valid addresses and skip
  // their loads and stores. With no return ahead of them, every kernel
  // argument can be fetched at once at the start instead of one scalar load
  // round trip after another.
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = static_cast<int>(block_order(blockIdx.x, gridDim.x, a.runs)) * TPB +
                   static_cast<int>(threadIdx.x) / kWave;
  const int tl_any = static_cast<int>(fast_div(static_cast<unsigned>(wave), a.by_chunks));
  const bool live = tl_any < a.tokens;
  const int tl = live ? tl_any : 0;
  const int chunk = live ? wave - tl * a.chunks : 0;
  const int token = a.token0 + tl;
  const int half = a.head_dim / 2;
  const int unit = NEOX ? half : a.head_dim;  // elements one lane group covers
  const int per_unit = unit / E;              // packets per unit (<= 64, host-checked)
  int j, hl, heads_per_iter;
  if (a.pu_shift >= 0) {
    j = lane & (per_unit - 1);
    hl = lane >> a.pu_shift;
    heads_per_iter = kWave >> a.pu_shift;
  } else {
    j = lane % per_unit;
    hl = lane / per_unit;
    heads_per_iter = kWave / per_unit;
  }
  const bool lane_live = live && hl < heads_per_iter;

  const int b = static_cast<int>(fast_div(static_cast<unsigned>(token), a.by_seq));
  const int s = token - b * a.seq;
  const int h01 = static_cast<int>(a.t0.heads + a.t1.heads);
  const int total = h01 + (CACHE ? static_cast<int>(a.t2.heads) : 0);
  const int base = chunk * ITERS * heads_per_iter;
  // The tensor of head h is chosen field by field, by value: the fields then
  // come from scalar kernel-argument loads and a per-lane select. Binding a
  // reference to the per-lane choice makes the compiler fetch the whole
  // descriptor with vector loads, a memory round trip that every wavefront
  // waits for before it can issue its first data load.
  const auto pick = [&](int h, const auto& f0, const auto& f1, const auto& f2) {
    return h < a.t0.heads ? f0 : ((CACHE && h >= h01) ? f2 : f1);
  };
  const auto head_in = [&](int h) -> int64_t {
    return h < a.t0.heads ? h : ((CACHE && h >= h01) ? h - h01 : h - a.t0.heads);
  };

  // Row of the tables and, in KV-cache mode, the cache slot of this token. A
  // token whose slot falls outside the cache writes no cache slot, and its q
  // rows are filled with NaN (table row 0 is read and replaced by NaN, so the
  // rotation yields NaN): the broken contract shows instead of stale memory.
  float c[NT], n[NT];
  int p = s;
  [[maybe_unused]] bool dropped = false;
  const auto load_tables = [&]() {
    if constexpr (CACHE) {
      const int64_t pp = *a.pos + s;
      dropped = pp < 0 || pp >= a.cache_len;
      p = dropped ? 0 : static_cast<int>(pp);
    }
    load_f32<TT, NT>(static_cast<const TT*>(a.cos) + p * a.st + j * NT, c);
    load_f32<TT, NT>(static_cast<const TT*>(a.sin) + p * a.st + j * NT, n);
    if constexpr (CACHE) {
      if (dropped) {
#pragma unroll
        for (int e = 0; e < NT; ++e) c[e] = n[e] = __builtin_nanf("");
      }
    }
  };
  // In KV-cache mode the source rows do not depend on the position, which is
  // a dependent scalar load: their loads are issued first, so the position's
  // round trip overlaps them instead of preceding them. Otherwise the table
  // row goes first, as the data loads' addresses need no memory read either.
  if constexpr (!CACHE) load_tables();
  P lo[ITERS], hi[ITERS];
  T* dst[ITERS];
  [[maybe_unused]] int64_t row_stride[ITERS];
  [[maybe_unused]] bool first[ITERS];
  [[maybe_unused]] bool copy[ITERS];
  // Each head group's addresses are formed right before its loads (forming
  // the destinations after all loads measured 0.8 points of peak slower at
  // (4, 2048)). In KV-cache mode the destination row of k and v is the cache
  // slot, known only once the position is read: the rest of the address is
  // formed here and the row added after.
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int h = base + it * heads_per_iter + hl;
    dst[it] = nullptr;
    if (lane_live && h < total) {
      const void* x = pick(h, a.t0.x, a.t1.x, a.t2.x);
      const int64_t sxb = pick(h, a.t0.sxb, a.t1.sxb, a.t2.sxb), sxs = pick(h, a.t0.sxs, a.t1.sxs, a.t2.sxs),
                    sxh = pick(h, a.t0.sxh, a.t1.sxh, a.t2.sxh);
      const int64_t hh = head_in(h);
      const T* src = static_cast<const T*>(x) + b * sxb + s * sxs + hh * sxh + j * E;
      void* y = pick(h, a.t0.y, a.t1.y, a.t2.y);
      const int64_t syb = pick(h, a.t0.syb, a.t1.syb, a.t2.syb), sys = pick(h, a.t0.sys, a.t1.sys, a.t2.sys),
                    syh = pick(h, a.t0.syh, a.t1.syh, a.t2.syh);
      if constexpr (CACHE) {
        dst[it] = static_cast<T*>(y) + b * syb + hh * syh + j * E;
        row_stride[it] = sys;
        first[it] = h < a.t0.heads;
        copy[it] = h >= h01;
      } else {
        dst[it] = static_cast<T*>(y) + b * syb + s * sys + hh * syh + j * E;
      }
      lo[it] = load_pack<T, E, true>(src);
      if constexpr (NEOX) hi[it] = load_pack<T, E, true>(src + half);
    }
  }
  if constexpr (CACHE) {
    load_tables();
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if (dst[it] == nullptr) continue;
      if (dropped && !first[it]) dst[it] = nullptr;  // no cache slot for this token
      else dst[it] += (first[it] ? s : p) * row_stride[it];
    }
  }
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    if (dst[it] == nullptr) continue;
    if constexpr (CACHE) {
      if (copy[it]) {
        store_pack<T, E, true>(dst[it], lo[it]);
        if constexpr (NEOX) store_pack<T, E, true>(dst[it] + half, hi[it]);
        continue;
      }
    }
    if constexpr (NEOX) {
      P olo, ohi;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float x0 = to_f32(lo[it].e[e]);
        const float x1 = to_f32(hi[it].e[e]);
        olo.e[e] = from_f32<T>(x0 * c[e] - x1 * n[e]);
        ohi.e[e] = from_f32<T>(x0 * n[e] + x1 * c[e]);
      }
      store_pack<T, E, true>(dst[it], olo);
      store_pack<T, E, true>(dst[it] + half, ohi);
    } else {
      P o;
#pragma unroll
      for (int i = 0; i < E / 2; ++i) {
        const float x0 = to_f32(lo[it].e[2 * i]);
        const float x1 = to_f32(lo[it].e[2 * i + 1]);
        o.e[2 * i] = from_f32<T>(x0 * c[i] - x1 * n[i]);
        o.e[2 * i + 1] = from_f32<T>(x0 * n[i] + x1 * c[i]);
      }
      store_pack<T, E, true>(dst[it], o);
    }
  }
}

// One lane per rotated pair; a grid-stride loop so any size fits one launch.
template <typename T, typename TT, bool NEOX, bool CACHE>
__global__ __launch_bounds__(256) void rope_scalar(RopeDev a) {
  const int half = a.head_dim / 2;
  const int64_t h01 = a.t0.heads + a.t1.heads;
  const int64_t total_heads = h01 + (CACHE ? a.t2.heads : 0);
  const int64_t pairs = a.total_tokens * total_heads * half;
  const int64_t p0 = CACHE ? *a.pos : 0;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < pairs;
       g += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = g % half;
    const int64_t th = g / half;
    const int64_t h = th % total_heads;
    const int64_t token = th / total_heads;
    const int64_t b = token / a.seq;
    const int64_t s = token - b * a.seq;
    const int64_t p = CACHE ? p0 + s : s;
    const bool first = h < a.t0.heads;
    const bool third = CACHE && h >= h01;
    // Outside the cache: no cache slot is written and q gets NaN (as rope_vec).
    const bool dropped = CACHE && (p < 0 || p >= a.cache_len);
    if (dropped && !first) continue;
    // Field by field, by value (scalar loads and a select; see rope_vec).
    const auto pick = [&](const auto& f0, const auto& f1, const auto& f2) { return first ? f0 : (third ? f2 : f1); };
    const int64_t hh = first ? h : (third ? h - h01 : h - a.t0.heads);
    const int64_t srow = (CACHE && !first) ? p : s;
    const T* src = static_cast<const T*>(pick(a.t0.x, a.t1.x, a.t2.x)) + b * pick(a.t0.sxb, a.t1.sxb, a.t2.sxb) +
                   s * pick(a.t0.sxs, a.t1.sxs, a.t2.sxs) + hh * pick(a.t0.sxh, a.t1.sxh, a.t2.sxh);
    T* dst = static_cast<T*>(pick(a.t0.y, a.t1.y, a.t2.y)) + b * pick(a.t0.syb, a.t1.syb, a.t2.syb) +
             srow * pick(a.t0.sys, a.t1.sys, a.t2.sys) + hh * pick(a.t0.syh, a.t1.syh, a.t2.syh);
    const int64_t ia = NEOX ? i : 2 * i;
    const int64_t ib = NEOX ? i + half : 2 * i + 1;
    if (third) {
      dst[ia] = src[ia];
      dst[ib] = src[ib];
      continue;
    }
    if (dropped) {
      dst[ia] = dst[ib] = from_f32<T>(__builtin_nanf(""));
      continue;
    }
    const float c = to_f32(static_cast<const TT*>(a.cos)[p * a.st + i]);
    const float n = to_f32(static_cast<const TT*>(a.sin)[p * a.st + i]);
    const float x0 = to_f32(src[ia]);
    const float x1 = to_f32(src[ib]);
    dst[ia] = from_f32<T>(x0 * c - x1 * n);
    dst[ib] = from_f32<T>(x0 * n + x1 * c);
  }
}

namespace {

RopeTensorDev to_dev(const RopeTensorArgs& t) {
  return RopeTensorDev{t.x, t.y, t.heads, t.sxb, t.sxs, t.sxh, t.syb, t.sys, t.syh};
}

constexpr int kWavesPerBlock = 4;
constexpr unsigned kRunsMinBlocks = 8192;
constexpr unsigned kRun = 128;
constexpr int64_t kWavesPerLaunch = int64_t(1) << 24;  // keeps grid work-items < 2^32

template <typename T, typename TT, bool NEOX, int ITERS, bool CACHE, int TPB = kWavesPerBlock>
hipError_t run_vec(RopeDev d, int64_t per_unit, hipStream_t stream) {
  const int64_t heads_per_wave = ITERS * (kWave / per_unit);
  d.chunks = static_cast<int>(ceil_div(d.t0.heads + d.t1.heads + (CACHE ? d.t2.heads : 0), heads_per_wave));
  d.by_chunks = make_fastdiv(static_cast<unsigned>(d.chunks));
  d.by_seq = make_fastdiv(static_cast<unsigned>(d.seq));
  d.pu_shift = (per_unit & (per_unit - 1)) == 0 ? __builtin_ctzll(per_unit) : -1;
  const int forced = g_rope_tuning.xcd_chunk;
  const bool one_tensor = d.t1.heads == 0 && !CACHE;
  const int64_t tokens_per_launch = std::max<int64_t>(1, kWavesPerLaunch / d.chunks);
  for (int64_t first = 0; first < d.total_tokens; first += tokens_per_launch) {
    RopeDev part = d;
    part.token0 = static_cast<int>(first);
    part.tokens = static_cast<int>(std::min(tokens_per_launch, d.total_tokens - first));
    const dim3 grid(static_cast<unsigned>(ceil_div(int64_t(part.tokens) * d.chunks, TPB)));
    // Launches of one tensor with at least kRunsMinBlocks workgroups hand
    // them to the XCDs in runs of kRun. Over five placements of the buffers
    // on MI355X (interleaved back-to-back timings, random spacers between
    // the input copies), q alone at (4, 2048) gained +0.3 to +1.6 points of
    // peak (fp16) and +0.8 to +1.1 (bf16) with runs of 128, while the fused
    // q+k launch lost 1.5-2.1 points with them (0.2-0.7 with runs of 32):
    // it keeps block order, as do the cache mode and smaller launches. Two
    // more boxes, four placements each, agreed: q alone +0.6 to +1.3 (box
    // means), q+k -0.3 to -1.8 with runs of 4, 32 or 128.
    unsigned chunk = 1;
    if (forced > 0) chunk = static_cast<unsigned>(forced);
    else if (one_tensor && grid.x >= kRunsMinBlocks) chunk = kRun;
    part.runs = make_xcd_runs(chunk);
    AKO_LAUNCH((rope_vec<T, TT, NEOX, ITERS, TPB, CACHE>), grid, dim3(kWave * TPB), 0,
               stream, part);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

// Head groups each wavefront rotates. Many short wavefronts keep the most
// independent 16-byte requests in flight per CU (measured on MI355X: one
// packet per lane per tensor row beats deep per-lane unrolling for pure
// streams), so the default is one group; ako_set_tuning(1, 2, n) overrides.
template <typename T, typename TT, bool NEOX>
hipError_t run_iters(const RopeDev& d, int64_t per_unit, hipStream_t stream) {
  const int forced_iters = g_rope_tuning.iters;
  const int iters = forced_iters > 0 ? forced_iters : 1;
  // Wavefronts per workgroup: one for launches of at most 2048 wavefronts
  // (decode), so that they spread over as many CUs as possible (graph-replayed
  // on MI355X, q of (64, 1, 32, 128): 2.10 us against 2.23 us with four);
  // four otherwise (no measurable difference at prefill sizes).
  int tpb = g_rope_tuning.tokens_per_block;
  if (tpb <= 0) {
    const int64_t heads = d.t0.heads + d.t1.heads + (d.pos != nullptr ? d.t2.heads : 0);
    const int64_t waves = d.total_tokens * ceil_div(heads, kWave / per_unit);
    tpb = waves <= 2048 ? 1 : kWavesPerBlock;
  }
  if (d.pos != nullptr) {
    return tpb == 1 ? run_vec<T, TT, NEOX, 1, true, 1>(d, per_unit, stream)
                    : run_vec<T, TT, NEOX, 1, true>(d, per_unit, stream);
  }
  if (iters <= 1) {
    switch (tpb) {
      case 1: return run_vec<T, TT, NEOX, 1, false, 1>(d, per_unit, stream);
      case 2: return run_vec<T, TT, NEOX, 1, false, 2>(d, per_unit, stream);
      case 8: return run_vec<T, TT, NEOX, 1, false, 8>(d, per_unit, stream);
      case 16: return run_vec<T, TT, NEOX, 1, false, 16>(d, per_unit, stream);
      default: return run_vec<T, TT, NEOX, 1, false>(d, per_unit, stream);
    }
  }
  if (iters <= 2) return run_vec<T, TT, NEOX, 2, false>(d, per_unit, stream);
  if (iters <= 4) return run_vec<T, TT, NEOX, 4, false>(d, per_unit, stream);
  return run_vec<T, TT, NEOX, 8, false>(d, per_unit, stream);
}

template <typename T, typename TT>
hipError_t run_typed(const RopeArgs& a, hipStream_t stream) {
  RopeDev d{to_dev(a.t0), to_dev(a.t1), to_dev(a.t2), a.pos, a.cache_len, a.cos, a.sin, 0, 0, 1,
            static_cast<int>(a.seq), static_cast<int>(a.head_dim), -1, a.st, a.batch * a.seq};
  if (a.vector_ok) {
    constexpr int E = 16 / sizeof(T);
    const int64_t unit = a.neox ? a.head_dim / 2 : a.head_dim;
    const int64_t per_unit = unit / E;
    return a.neox ? run_iters<T, TT, true>(d, per_unit, stream)
                  : run_iters<T, TT, false>(d, per_unit, stream);
  }
  const int64_t heads = a.t0.heads + a.t1.heads + (a.pos != nullptr ? a.t2.heads : 0);
  const int64_t pairs = d.total_tokens * heads * (a.head_dim / 2);
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(pairs, 256), 1 << 16));
  const dim3 grid(blocks), block(256);
  if (a.pos != nullptr) {
    if (a.neox) AKO_LAUNCH((rope_scalar<T, TT, true, true>), grid, block, 0, stream, d);
    else AKO_LAUNCH((rope_scalar<T, TT, false, true>), grid, block, 0, stream, d);
  } else {
    if (a.neox) AKO_LAUNCH((rope_scalar<T, TT, true, false>), grid, block, 0, stream, d);
    else AKO_LAUNCH((rope_scalar<T, TT, false, false>), grid, block, 0, stream, d);
  }
  return hipGetLastError();
}

template <typename T>
hipError_t run_table(const RopeArgs& a, hipStream_t stream) {
  switch (a.table_dtype) {
    case kF32: return run_typed<T, float>(a, stream);
    case kF16: return run_typed<T, _Float16>(a, stream);
    case kBF16: return run_typed<T, __bf16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_rope(const RopeArgs& a, hipStream_t stream) {
  switch (a.dtype) {
    case kF32: return run_table<float>(a, stream);
    case kF16: return run_table<_Float16>(a, stream);
    case kBF16: return run_table<__bf16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ako

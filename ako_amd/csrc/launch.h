// Internal launcher interface between the C ABI layer (abi.hip) and the
// kernel translation units. Arguments reaching these functions have already
// been validated by abi.hip: sizes positive, pointers non-null and aligned as
// the chosen path requires, strides consistent.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace ako {

// A start/stop event pair armed by ako_time_next_launch on one host thread.
// The next kernel launch that thread makes through AKO_LAUNCH takes the pair
// (and disarms it): it goes out through hipExtLaunchKernelGGL, which binds
// both events to the dispatch itself, so their elapsed time is the kernel's
// own start-to-end time, with no marker packets queued around it. Launches
// without an armed pair are plain hipLaunchKernelGGL launches.
struct ArmedEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
inline ArmedEvents& armed_events() {
  thread_local ArmedEvents pair;
  return pair;
}
inline ArmedEvents take_armed_events() {
  ArmedEvents& slot = armed_events();
  const ArmedEvents taken = slot;
  slot = ArmedEvents{};
  return taken;
}

// hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...), or the same
// launch carrying the thread's armed event pair. A kernel name with template
// arguments goes in parentheses, as for hipLaunchKernelGGL.
#define AKO_LAUNCH(kernel, grid, block, lds, stream, ...)                                              \
  do {                                                                                                 \
    const ::ako::ArmedEvents ako_events_ = ::ako::take_armed_events();                                 \
    if (ako_events_.start != nullptr)                                                                  \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, ako_events_.start, ako_events_.stop, 0u, \
                            __VA_ARGS__);                                                              \
    else                                                                                               \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                               \
  } while (0)

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

inline int dtype_bytes(int dt) { return dt == kF32 ? 4 : 2; }

// Launch-shape overrides set through ako_set_tuning (0 = heuristic). Every
// key is an atomic int: ako_set_tuning may run on any host thread while other
// threads launch, and each read in a launcher sees the value before or after
// a concurrent set (a launch concurrent with several sets may mix them).
using TuningKey = std::atomic<int>;
struct RmsTuning {
  TuningKey waves_per_row{0};    // key 1
  TuningKey vecs_per_thread{0};  // key 2
  TuningKey force_stream{0};     // key 3: 1 = always use the two-pass kernel
  TuningKey lds_reserve{0};      // key 4: bytes of LDS reserved per workgroup (caps rows in flight per CU)
  TuningKey row_order{0};        // key 5: 1 = rows in block order, 2 = XCD-blocked order
  TuningKey xcd_chunk{0};        // key 6: consecutive blocks per XCD run in XCD-blocked order (0 = n / 8)
  TuningKey max_blocks{0};       // key 7: cap on workgroups per launch (0 = 2^31 work-items)
  TuningKey early_weights{0};    // key 8: 1 = weights after the row's loads return, 2 = with them (0 = by launch size)
  TuningKey pipeline{0};         // key 9: 1 = never the pipelined persistent kernel, 2 = whenever eligible (0 = heuristic)
  TuningKey pipe_blocks_per_cu{0};  // key 10: workgroups per CU in the pipelined grid (0 = 16 wavefronts per CU)
  TuningKey load_groups{0};      // key 11: residual (16, 2) rows: 1 = both packets per load group, 2 = one (0 = one with write-through stores, else by dtype)
  TuningKey write_through{0};    // key 12: (16, 2) and (16, 1) rows: 1 = non-temporal stores, 2 = write-through stores (0 = write-through on (16, 2) launches of many rows)
};
struct RopeTuning {
  TuningKey tokens_per_block{0};  // key 1: wavefronts per workgroup (1, 2, 4, 8 or 16; one group per wavefront)
  TuningKey iters{0};             // key 2: head chunks unrolled per loop trip
  TuningKey xcd_chunk{0};         // key 3: consecutive workgroups per XCD run (1 = block order; 0 = runs of 128 for one tensor from 8192 workgroups)
};
struct SwigluTuning {
  TuningKey vecs_per_thread{0};  // key 1: packets per lane (1, 2, 4 or 8)
  TuningKey xcd_chunk{0};        // key 2: consecutive workgroups per XCD run in dense launches (1 = block order; 0 = runs of 4 for launches of 2048-65535 workgroups)
};
extern RmsTuning g_rms_tuning;
extern RopeTuning g_rope_tuning;
extern SwigluTuning g_swiglu_tuning;

struct RmsArgs {
  const void* x;
  const void* r;  // residual input (residual variant only)
  const void* w;
  void* y;
  void* rout;     // residual output (residual variant only)
  int64_t rows;
  int64_t hidden;
  int64_t sx, sr, sy, srout;  // row strides, elements
  float eps;
  int dtype;
  int w_dtype;
  bool residual;
  bool vector_ok;  // 16-byte packets are aligned for every row
};
hipError_t launch_rmsnorm(const RmsArgs& a, hipStream_t stream);

// One rank's slice of a hidden-sharded row (tensor parallelism). partial:
// x (+ r, rounded, to rout) -> fp32 sum of squares per row in `partial`.
// apply: x holds s, `total` the all-reduced sums, y = s * rsqrt(total/H + eps) * w.
struct RmsShardArgs {
  const void* x;
  const void* r;
  const void* w;
  void* y;
  void* rout;
  float* partial;
  const float* total;
  int64_t rows;
  int64_t shard;   // elements of the slice
  int64_t hidden;  // full row length H (apply)
  int64_t sx, sr, sy, srout;
  float eps;
  int dtype;
  int w_dtype;
  bool residual;
  bool vector_ok;
};
hipError_t launch_rmsnorm_shard_partial(const RmsShardArgs& a, hipStream_t stream);
hipError_t launch_rmsnorm_shard_apply(const RmsShardArgs& a, hipStream_t stream);

struct RopeTensorArgs {
  const void* x;
  void* y;
  int64_t heads;
  int64_t sxb, sxs, sxh;
  int64_t syb, sys, syh;
};
struct RopeArgs {
  RopeTensorArgs t0;
  RopeTensorArgs t1;  // heads == 0 when only one tensor is rotated
  // KV-cache mode (pos != nullptr): token s sits at position p = *pos + s; the
  // tables are read at row p, t1's output row is slot p (rotated keys into the
  // cache) and t2 is copied unrotated to slot p of its output (values). Tokens
  // with p outside [0, cache_len) are not written.
  RopeTensorArgs t2;
  const int64_t* pos;
  int64_t cache_len;
  const void* cos;
  const void* sin;
  int64_t batch, seq, head_dim;
  int64_t st;  // table row stride, elements
  int dtype, table_dtype;
  bool neox;
  bool vector_ok;
};
hipError_t launch_rope(const RopeArgs& a, hipStream_t stream);

struct SwigluArgs {
  const void* g;
  const void* u;
  void* y;
  int64_t rows, n;
  int64_t sg, su, sy;
  int dtype;
  bool contiguous;  // all three are one dense [rows * n] block
  bool vector_ok;
};
hipError_t launch_swiglu(const SwigluArgs& a, hipStream_t stream);

}  // namespace ako

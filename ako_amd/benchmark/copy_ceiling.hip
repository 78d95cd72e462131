// Size-dependent streaming ceiling of one GPU: the per-launch time of a plain
// device copy (16-byte packets, one per lane, non-temporal loads and stores)
// at given byte counts, with cold buffers.
//
// The copy's fraction of the HBM peak at a cell's byte count is the reference
// each hot-path cell is compared with: what the plainest stream of the same
// bytes reaches on the same box. It is not a strict bound (a kernel that
// orders its reads and writes differently can pass it, as the pipelined
// RMSNorm does by a few percent). It falls with size because every launch
// pays a roughly fixed ramp-up and drain.
//
// Usage: copy_ceiling [bytes_per_buffer ...]   (default: the hot-path cell sizes)
// Prints one JSON object per size, block shape and store policy:
//   {"bytes_per_buffer": N, "traffic_bytes": 2N, "block": 256, "store": "nt",
//    "us": t, "gbps": 2N/t, "frac": gbps/8000}
// Buffers rotate through a 2 GiB source pool and a 2 GiB destination pool, so
// consecutive launches never find their data in the 256 MB MALL or the L2s.
// The 25 launches of a size are queued back to back, each with its own pair
// of events bound to the launch (hipExtLaunchKernelGGL: the events take the
// dispatch's own start and end, with no marker packets between the copies),
// behind a short spin kernel that keeps the device busy while they are
// queued, and the stream is synchronised once at the end (as bench.py times
// each launch); the median of the last 22 is reported as "us". The same 22
// launches are then queued again between one pair of events around all of
// them (as bench.py times its extra cells), and the mean is reported as
// "b2b_us".
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                         \
  do {                                                                                   \
    hipError_t err_ = (x);                                                               \
    if (err_ != hipSuccess) {                                                            \
      std::fprintf(stderr, "copy_ceiling: %s at line %d\n", hipGetErrorString(err_), __LINE__); \
      std::exit(1);                                                                      \
    }                                                                                    \
  } while (0)

// STORE 0: the store carries the nt bit (__builtin_nontemporal_store), as the
// hot-path kernels' stores do. STORE 1: sc1 and nt, which makes the store
// agent-coherent (written through the XCD's L2). A plain copy runs 3-4% faster
// with it; kernels that read more than they write do not (measured), so the
// kernels keep nt, but the faster copy is the ceiling reported. The s_nop is
// the wait state a store of more than 64 bits of data needs before a VALU may
// overwrite its data registers, which the compiler cannot see inside the asm.
template <int BLOCK, int STORE>
__global__ __launch_bounds__(BLOCK) void copy_packets(const u32x4* __restrict__ a, u32x4* __restrict__ b, long n) {
  const long i = (long)blockIdx.x * BLOCK + threadIdx.x;
  if (i < n) {
    const u32x4 v = __builtin_nontemporal_load(a + i);
    if constexpr (STORE == 0) {
      __builtin_nontemporal_store(v, b + i);
    } else {
      asm volatile("global_store_dwordx4 %0, %1, off sc1 nt\n\ts_nop 0" : : "v"(b + i), "v"(v));
    }
  }
}

// One copy launch; with events, they are bound to it (its start and end).
template <int BLOCK, int STORE>
void launch_copy(long n, const u32x4* a, u32x4* b, hipEvent_t start, hipEvent_t stop) {
  const dim3 grid((n + BLOCK - 1) / BLOCK);
  if (start != nullptr) {
    hipExtLaunchKernelGGL((copy_packets<BLOCK, STORE>), grid, dim3(BLOCK), 0, 0, start, stop, 0u, a, b, n);
  } else {
    hipLaunchKernelGGL((copy_packets<BLOCK, STORE>), grid, dim3(BLOCK), 0, 0, a, b, n);
  }
}

// Keeps one wavefront busy for `cycles` shader-clock cycles, with no memory
// traffic: queued ahead of a timed region so that its first event is reached
// with the first timed launch already queued (on an idle device the event
// completes at once and the host's submission time of the first launch
// would be timed). The loop ends once the clock has advanced that far.
__global__ void spin(long long cycles) {
  const long long t0 = clock64();
  while (clock64() - t0 < cycles) __builtin_amdgcn_s_sleep(1);
}

static constexpr long kPool = 1L << 31;
static constexpr double kPeakGBs = 8000.0;

int main(int argc, char** argv) {
  std::vector<long> sizes;
  for (int i = 1; i < argc; ++i) sizes.push_back(std::atol(argv[i]));
  if (sizes.empty()) {
    // Half the algorithmic bytes of each prefill cell (a copy of N bytes moves 2N):
    // RoPE (4, 2048, h, 128) half precision, k (h = 8), q (h = 32) and q + k in one
    // launch; RMSNorm, 16384 rows of 4096 / 8192 / 16384 half elements (the
    // residual variant moves twice the plain one); SwiGLU bf16 M x 14336 at
    // M = 4096 and 16384 (three streams, so only roughly a copy).
    sizes = {17039360L, 67371008L, 84148224L, 128L << 20, 176160768L, 256L << 20, 512L << 20, 704643072L, 1L << 30};
  }
  for (long bytes : sizes) {
    if (bytes < 16 || bytes > kPool || bytes % 16 != 0) {
      std::fprintf(stderr, "copy_ceiling: size %ld must be a multiple of 16 in [16, %ld]\n", bytes, kPool);
      return 2;
    }
  }
  char* src = nullptr;
  char* dst = nullptr;
  CHECK(hipMalloc(&src, kPool));
  CHECK(hipMalloc(&dst, kPool));
  CHECK(hipMemset(src, 1, kPool));
  CHECK(hipMemset(dst, 0, kPool));
  constexpr int kReps = 25, kWarm = 3;
  constexpr long long kLeadCycles = 200000;  // 80-140 us at MI355X clocks
  hipEvent_t start[kReps], stop[kReps];
  for (int i = 0; i < kReps; ++i) {
    CHECK(hipEventCreate(&start[i]));
    CHECK(hipEventCreate(&stop[i]));
  }
  for (long bytes : sizes) {
    const long n = bytes / 16;
    const long slots = kPool / bytes;  // >= 1; slot s spans [s*bytes, (s+1)*bytes) of each pool
    for (int variant = 0; variant < 4; ++variant) {
      const int block = variant % 2 ? 1024 : 256;
      const int store = variant / 2;
      const auto launch = [&](int rep, hipEvent_t ev0, hipEvent_t ev1) {
        const long off = (rep % slots) * bytes;
        const u32x4* a = reinterpret_cast<const u32x4*>(src + off);
        u32x4* b = reinterpret_cast<u32x4*>(dst + off);
        if (variant == 0) launch_copy<256, 0>(n, a, b, ev0, ev1);
        if (variant == 1) launch_copy<1024, 0>(n, a, b, ev0, ev1);
        if (variant == 2) launch_copy<256, 1>(n, a, b, ev0, ev1);
        if (variant == 3) launch_copy<1024, 1>(n, a, b, ev0, ev1);
        CHECK(hipGetLastError());
      };
      hipLaunchKernelGGL(spin, dim3(1), dim3(64), 0, 0, kLeadCycles);
      CHECK(hipGetLastError());
      for (int rep = 0; rep < kReps; ++rep) launch(rep, start[rep], stop[rep]);
      CHECK(hipDeviceSynchronize());
      // Back to back: the timed launches again, one event pair around them all,
      // behind the spin and the kWarm untimed launches (their own slots), so
      // the first timed launch follows copies as every later one does.
      hipLaunchKernelGGL(spin, dim3(1), dim3(64), 0, 0, kLeadCycles);
      CHECK(hipGetLastError());
      for (int rep = 0; rep < kWarm; ++rep) launch(rep, nullptr, nullptr);
      CHECK(hipEventRecord(start[0]));
      for (int rep = kWarm; rep < kReps; ++rep) launch(rep, nullptr, nullptr);
      CHECK(hipEventRecord(stop[0]));
      CHECK(hipDeviceSynchronize());
      float b2b_ms = 0.f;
      CHECK(hipEventElapsedTime(&b2b_ms, start[0], stop[0]));
      const double b2b_us = 1e3 * b2b_ms / (kReps - kWarm);
      std::vector<float> ms_list;
      for (int rep = kWarm; rep < kReps; ++rep) {
        float ms = 0.f;
        CHECK(hipEventElapsedTime(&ms, start[rep], stop[rep]));
        ms_list.push_back(ms);
      }
      std::sort(ms_list.begin(), ms_list.end());
      const double us = 1e3 * ms_list[ms_list.size() / 2];
      const double gbps = 2.0 * bytes / (us * 1e-6) / 1e9;
      const double b2b_gbps = 2.0 * bytes / (b2b_us * 1e-6) / 1e9;
      std::printf("{\"bytes_per_buffer\": %ld, \"traffic_bytes\": %ld, \"block\": %d, \"store\": \"%s\", "
                  "\"us\": %.2f, \"gbps\": %.1f, \"frac\": %.4f, \"b2b_us\": %.2f, \"b2b_gbps\": %.1f, "
                  "\"b2b_frac\": %.4f}\n",
                  bytes, 2 * bytes, block, store ? "sc1 nt" : "nt", us, gbps, gbps / kPeakGBs, b2b_us, b2b_gbps,
                  b2b_gbps / kPeakGBs);
      std::fflush(stdout);
    }
  }
  CHECK(hipFree(src));
  CHECK(hipFree(dst));
  return 0;
}

/*
 * ako_hip.h - C ABI of the MI355X (gfx950) AKO candidate kernels.
 *
 * One shared library, libako_hip.so, exports the entry points below. They
 * take plain device pointers, element counts and strides, a dtype code and a
 * hipStream_t passed as void*. No PyTorch (or any C++) type crosses this
 * boundary, so the library can be bound from ctypes, cgo or JNI alike.
 *
 * Each entry point replaces one Triton candidate of the reference
 * (Farx1/AKO); the citation next to each declaration names the host wrapper
 * and kernel whose contract it takes over.
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers (hipMalloc'd or from a caching allocator).
 *   - Strides are in ELEMENTS, not bytes. The innermost dimension (hidden,
 *     head_dim, n) must be contiguous.
 *   - Outputs must not overlap any input; overlapping ranges are rejected.
 *   - Work is enqueued on `stream` (NULL = the default stream) and the call
 *     returns without synchronising. Launch errors are reported; errors that
 *     happen later on the device surface at the caller's next sync.
 *   - Arithmetic is fp32 internally for every storage dtype; results are
 *     rounded to the output dtype with round-to-nearest-even.
 *   - Return value: AKO_OK (0) or a nonzero ako_status_t; ako_last_error()
 *     then returns a message (thread-local, valid until the next call on the
 *     same thread).
 *   - Empty work (rows == 0, hidden == 0, ...) returns AKO_OK and launches
 *     nothing.
 */
#ifndef AKO_HIP_H
#define AKO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AKO_ABI_VERSION 1

typedef enum {
  AKO_DTYPE_F32 = 0,
  AKO_DTYPE_F16 = 1,
  AKO_DTYPE_BF16 = 2
} ako_dtype_t;

typedef enum {
  AKO_OK = 0,
  AKO_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, bad stride, overlap */
  AKO_ERR_UNSUPPORTED = 2,      /* dtype combination or style not provided      */
  AKO_ERR_HIP = 3,              /* the HIP runtime reported an error            */
  AKO_ERR_NO_DEVICE = 4         /* no usable GPU in this process                 */
} ako_status_t;

typedef enum {
  AKO_ROPE_NEOX = 0,        /* pairs (i, i + head_dim/2) */
  AKO_ROPE_INTERLEAVED = 1  /* pairs (2i, 2i + 1)        */
} ako_rope_style_t;

/* Library identity: AKO_ABI_VERSION, and the HIP runtime version
 * (hipRuntimeGetVersion) of the runtime this library is bound to. */
int ako_abi_version(void);
int ako_hip_runtime_version(void);
const char* ako_build_info(void);
const char* ako_last_error(void);

/*
 * Identity of GPU `device` for the selection cache key, written into buf as
 * one NUL-terminated line of key=value fields separated by ';':
 *   name=<hipDeviceProp_t.name>;arch=<gcnArchName>;cus=<CUs>;
 *   clock_khz=<peak engine clock>;mem_bytes=<HBM bytes>;hip_driver=<hipDriverGetVersion>
 * Replaces the device-name probe of ako/dispatcher/hardware.py:134-193 (CUDA
 * runtime attributes and nvidia-smi). The marketing name that HIP reports can
 * be a generic "AMD Radeon Graphics" for every part, so callers key by the
 * other fields too. Returns AKO_ERR_INVALID_ARGUMENT when buf is too small.
 */
int ako_device_identity(int device, char* buf, int64_t buf_len);

/*
 * RMSNorm over the last dimension:
 *   y[r, :] = to_dtype( (x[r, :] * rsqrt(sum(x[r, :]^2) / hidden + eps)) * w[:] )
 * x, y: dtype; w: w_dtype (== dtype, or AKO_DTYPE_F32).
 * Replaces rmsnorm_triton + _rmsnorm_kernel_impl
 * (ako/ops/rmsnorm_triton.py:56-81, 139-157). Unlike the reference there is
 * no hidden-size limit (the reference raised above 65536,
 * ako/ops/rmsnorm_triton.py:28,130-133).
 */
int ako_rmsnorm_fwd(const void* x, const void* w, void* y,
                    int64_t rows, int64_t hidden,
                    int64_t x_row_stride, int64_t y_row_stride,
                    float eps, int dtype, int w_dtype, void* stream);

/*
 * Residual-add + RMSNorm:
 *   s = to_dtype(x + residual)       (the sum is rounded to the storage dtype)
 *   residual_out = s
 *   y = RMSNorm(s, w, eps)
 * Replaces rmsnorm_residual_triton + _rmsnorm_residual_kernel_impl
 * (ako/ops/rmsnorm_triton.py:83-117, 160-192) and matches the unfused
 * reference ako/ops/rmsnorm_ref.py:26-50.
 */
int ako_rmsnorm_residual_fwd(const void* x, const void* residual, const void* w,
                             void* y, void* residual_out,
                             int64_t rows, int64_t hidden,
                             int64_t x_row_stride, int64_t r_row_stride,
                             int64_t y_row_stride, int64_t rout_row_stride,
                             float eps, int dtype, int w_dtype, void* stream);

/*
 * RMSNorm of a row whose hidden dimension is split over tensor-parallel
 * ranks: the per-rank halves of a fused all-reduce + residual + RMSNorm. The
 * reference has no tensor parallelism, so neither has a counterpart there;
 * together they compute rmsnorm_residual_ref / rmsnorm_ref
 * (ako/ops/rmsnorm_ref.py:8-50) on the whole row, up to the order of the
 * fp32 sum of squares:
 *   partial:  s = x (+ residual, rounded to dtype, written to residual_out;
 *             both NULL for plain RMSNorm), partial_ss[row] = sum of s^2 over
 *             the rank's `shard` elements (fp32);
 *   (the caller sums partial_ss over the ranks, e.g. one all-reduce)
 *   apply:    y = to_dtype((s * rsqrt(total_ss[row] * (1/hidden) + eps)) * w)
 *             on the rank's slice, with `hidden` the full row length.
 * Row strides in elements; partial_ss / total_ss hold `rows` floats.
 */
int ako_rmsnorm_shard_partial_fwd(const void* x, const void* residual, void* residual_out,
                                  float* partial_ss, int64_t rows, int64_t shard,
                                  int64_t x_row_stride, int64_t r_row_stride,
                                  int64_t rout_row_stride, int dtype, void* stream);
int ako_rmsnorm_shard_apply_fwd(const void* s, const void* w, const float* total_ss, void* y,
                                int64_t rows, int64_t shard, int64_t hidden,
                                int64_t s_row_stride, int64_t y_row_stride, float eps,
                                int dtype, int w_dtype, void* stream);

/*
 * Rotary position embedding of x[batch, seq, heads, head_dim]:
 *   for each pair (a, b) of a head at position s, with c = cos[s, i],
 *   n = sin[s, i]:   a' = a*c - b*n,   b' = a*n + b*c     (fp32)
 * cos/sin: [seq, head_dim/2] rows `table_row_stride` apart, dtype
 * `table_dtype` (F32, F16 or BF16, independent of x's dtype).
 * x strides (batch, seq, head) and y strides likewise, in elements.
 * Replaces rope_triton + _rope_kernel_impl (ako/ops/rope_triton.py:32-80,
 * 97-156); semantics of ako/ops/rope_ref.py:73-107.
 */
int ako_rope_fwd(const void* x, const void* cos_table, const void* sin_table, void* y,
                 int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                 int64_t x_stride_b, int64_t x_stride_s, int64_t x_stride_h,
                 int64_t y_stride_b, int64_t y_stride_s, int64_t y_stride_h,
                 int64_t table_row_stride,
                 int dtype, int table_dtype, int style, void* stream);

/*
 * RoPE of a query/key pair sharing the tables, in ONE launch (the reference
 * runs two, ako/ops/rope.py:45-58). q is [batch, seq, q_heads, head_dim],
 * k is [batch, seq, k_heads, head_dim]; strides as in ako_rope_fwd.
 */
int ako_rope_qk_fwd(const void* q, const void* k, const void* cos_table, const void* sin_table,
                    void* q_out, void* k_out,
                    int64_t batch, int64_t seq, int64_t q_heads, int64_t k_heads,
                    int64_t head_dim,
                    const int64_t* q_strides, const int64_t* k_strides,
                    const int64_t* q_out_strides, const int64_t* k_out_strides,
                    int64_t table_row_stride,
                    int dtype, int table_dtype, int style, void* stream);

/*
 * RoPE of a query/key pair with the rotated keys (and the values, copied)
 * written straight into a KV cache, in ONE launch. This is the fused consumer
 * the reference's decoder performs as rope(q), rope(k) and a cache append
 * (ako/models/decoder.py:173-177, KVCache.update at :84-93).
 *   position of token s:  p = *pos + s   (pos: one int64 in device memory,
 *                                         read by the kernel, so a captured
 *                                         launch follows a moving position)
 *   q_out[b, s, h]      = rope(q[b, s, h], row p of cos/sin)
 *   k_cache[b, h, slot p] = rope(k[b, s, h], row p)
 *   v_cache[b, h, slot p] = v[b, s, h]          (v and v_cache may both be NULL)
 * q/k/v/q_out strides are (batch, seq, head); cache_strides (batch, slot,
 * head) are shared by both caches, in elements. The tables hold table_rows
 * >= cache_len rows. A token whose p falls outside [0, cache_len) writes no
 * cache slot, and its q_out rows are filled with NaN; keeping
 * *pos + seq <= cache_len is the caller's contract (the reference's unfused
 * composition raises an index error there, which a position held in device
 * memory cannot do).
 */
int ako_rope_qk_cache_fwd(const void* q, const void* k, const void* v,
                          const void* cos_table, const void* sin_table,
                          void* q_out, void* k_cache, void* v_cache, const int64_t* pos,
                          int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads,
                          int64_t head_dim,
                          const int64_t* q_strides, const int64_t* k_strides,
                          const int64_t* v_strides, const int64_t* q_out_strides,
                          const int64_t* cache_strides,
                          int64_t cache_len, int64_t table_rows, int64_t table_row_stride,
                          int dtype, int table_dtype, int style, void* stream);

/*
 * SwiGLU activation: y = to_dtype( silu(gate) * up ), silu(g) = g / (1 + e^-g),
 * over [rows, n] with row strides in elements.
 * Replaces swiglu_triton + _swiglu_kernel_impl
 * (ako/ops/swiglu_triton.py:27-81); semantics of ako/ops/swiglu_ref.py:16-32.
 * No width limit (the reference raised above 65536).
 */
int ako_swiglu_fwd(const void* gate, const void* up, void* y,
                   int64_t rows, int64_t n,
                   int64_t gate_row_stride, int64_t up_row_stride, int64_t y_row_stride,
                   int dtype, void* stream);

/*
 * Launch-shape override for tuning sweeps and tests (no counterpart in the
 * reference, whose Triton autotuner explored num_warps itself); production
 * callers leave it alone. op: 0 = rmsnorm and rmsnorm_residual, 1 = rope,
 * 2 = swiglu. key/value pairs are documented in the kernel sources; value 0
 * restores the built-in heuristic. Process-wide. Each key is an atomic int,
 * so the call is safe from any host thread: a launch that runs concurrently
 * sees each key's value from before or after the call (a launch concurrent
 * with several calls may mix their values).
 */
int ako_set_tuning(int op, int key, int value);

/*
 * Timing hook for benchmarks (no counterpart in the reference, which timed
 * through Triton's do_bench): arms two HIP events for the next kernel launch
 * that the calling host thread makes through any entry point above. That
 * launch goes out through hipExtLaunchKernelGGL with the pair, which binds
 * both events to the dispatch itself: hipEventElapsedTime(start, stop) is
 * then the kernel's own start-to-end time, the figure a kernel trace reports,
 * without the marker packets that an hipEventRecord on each side would queue
 * around it. The events are the caller's (hipEventCreate, timing enabled);
 * an entry point that makes several launches (inputs past 2^31 work-items)
 * times its first. Arming replaces a pair that no launch has taken. Do
 * not arm a pair while the thread captures a stream into a graph: the next
 * launch takes it whether or not it is captured.
 * start and stop both NULL disarms: the return value is then 1 when a pair
 * was still armed (no launch took it), else AKO_OK. Exactly one NULL is
 * AKO_ERR_INVALID_ARGUMENT.
 */
int ako_time_next_launch(void* start_event, void* stop_event);

#ifdef __cplusplus
}
#endif

#endif /* AKO_HIP_H */

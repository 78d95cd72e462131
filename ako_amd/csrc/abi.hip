// The C ABI (include/ako_hip.h): argument validation, status codes, and the
// hand-off to the kernel launchers. Validation runs entirely on the host and
// before any HIP call, so every rejection path is testable on a machine
// without a GPU.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <limits>
#include <string>

#include "ako_hip.h"
#include "launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return AKO_OK;
  if (err == hipErrorNoDevice || err == hipErrorInvalidDevice)
    return fail(AKO_ERR_NO_DEVICE, "%s: %s", what, hipGetErrorString(err));
  return fail(AKO_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

bool valid_dtype(int dt) { return dt == AKO_DTYPE_F32 || dt == AKO_DTYPE_F16 || dt == AKO_DTYPE_BF16; }

const char* dtype_name(int dt) {
  switch (dt) {
    case AKO_DTYPE_F32: return "f32";
    case AKO_DTYPE_F16: return "f16";
    case AKO_DTYPE_BF16: return "bf16";
    default: return "?";
  }
}

bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

// Byte range [lo, hi) spanned by `count` rows of `width` elements, `stride`
// apart. `ok` is false when the extent exceeds 2^56 bytes or wraps the address
// space (sizes no allocation can have); the arithmetic is done in 128 bits so
// that such arguments cannot wrap into a small, plausible-looking span.
constexpr __int128 kMaxSpanBytes = static_cast<__int128>(1) << 56;

struct Span {
  uintptr_t lo = 0, hi = 0;
  bool ok = true;
};

Span span_bytes(const void* p, __int128 bytes) {
  Span s;
  s.lo = reinterpret_cast<uintptr_t>(p);
  if (bytes < 0 || bytes > kMaxSpanBytes) {
    s.ok = false;
    s.hi = s.lo;
    return s;
  }
  s.hi = s.lo + static_cast<uintptr_t>(bytes);
  s.ok = s.hi >= s.lo;
  return s;
}

Span span_2d(const void* p, int64_t rows, int64_t width, int64_t stride, int elem) {
  const __int128 last = static_cast<__int128>(rows - 1) * stride + width;
  return span_bytes(p, last * elem);
}

bool overlap(const Span& a, const Span& b) { return a.lo < b.hi && b.lo < a.hi; }

constexpr int64_t kMaxInt = std::numeric_limits<int32_t>::max();

}  // namespace

extern "C" {

int ako_abi_version(void) { return AKO_ABI_VERSION; }

int ako_hip_runtime_version(void) {
  int v = 0;
  if (hipRuntimeGetVersion(&v) != hipSuccess) return -1;
  return v;
}

const char* ako_build_info(void) {
  static const std::string info = std::string("ako_hip abi=") + std::to_string(AKO_ABI_VERSION) +
                                  " arch=gfx950 hip_headers=" + std::to_string(HIP_VERSION);
  return info.c_str();
}

const char* ako_last_error(void) { return g_last_error.c_str(); }

int ako_device_identity(int device, char* buf, int64_t buf_len) {
  const char* fn = "ako_device_identity";
  if (buf == nullptr || buf_len <= 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: no output buffer", fn);
  hipDeviceProp_t props;
  const hipError_t err = hipGetDeviceProperties(&props, device);
  if (err != hipSuccess) return hip_status(err, fn);
  int driver = 0;
  if (hipDriverGetVersion(&driver) != hipSuccess) driver = -1;
  props.name[sizeof(props.name) - 1] = '\0';
  props.gcnArchName[sizeof(props.gcnArchName) - 1] = '\0';
  const int n = std::snprintf(buf, static_cast<size_t>(buf_len),
                              "name=%s;arch=%s;cus=%d;clock_khz=%d;mem_bytes=%llu;hip_driver=%d", props.name,
                              props.gcnArchName, props.multiProcessorCount, props.clockRate,
                              static_cast<unsigned long long>(props.totalGlobalMem), driver);
  if (n < 0 || n >= buf_len) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: buffer of %lld bytes is too small", fn,
                                         static_cast<long long>(buf_len));
  return AKO_OK;
}

int ako_time_next_launch(void* start_event, void* stop_event) {
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(AKO_ERR_INVALID_ARGUMENT, "ako_time_next_launch: start and stop must both be set or both be NULL");
  ako::ArmedEvents& slot = ako::armed_events();
  if (start_event == nullptr) {
    const bool pending = slot.start != nullptr;
    slot = ako::ArmedEvents{};
    return pending ? 1 : AKO_OK;
  }
  slot.start = static_cast<hipEvent_t>(start_event);
  slot.stop = static_cast<hipEvent_t>(stop_event);
  return AKO_OK;
}

int ako_set_tuning(int op, int key, int value) {
  if (value < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "tuning value must be >= 0, got %d", value);
  switch (op) {
    case 0:
      if (key == 1) { ako::g_rms_tuning.waves_per_row = value; return AKO_OK; }
      if (key == 2) { ako::g_rms_tuning.vecs_per_thread = value; return AKO_OK; }
      if (key == 3) { ako::g_rms_tuning.force_stream = value; return AKO_OK; }
      if (key == 4) {
        if (value > 160 * 1024) return fail(AKO_ERR_INVALID_ARGUMENT, "LDS reserve above 160 KiB");
        ako::g_rms_tuning.lds_reserve = value;
        return AKO_OK;
      }
      if (key == 5) {
        if (value > 2) return fail(AKO_ERR_INVALID_ARGUMENT, "row order must be 0, 1 or 2");
        ako::g_rms_tuning.row_order = value;
        return AKO_OK;
      }
      if (key == 6) { ako::g_rms_tuning.xcd_chunk = value; return AKO_OK; }
      if (key == 7) { ako::g_rms_tuning.max_blocks = value; return AKO_OK; }
      if (key == 8) {
        if (value > 2) return fail(AKO_ERR_INVALID_ARGUMENT, "early weights must be 0, 1 or 2");
        ako::g_rms_tuning.early_weights = value;
        return AKO_OK;
      }
      if (key == 9) {
        if (value > 2) return fail(AKO_ERR_INVALID_ARGUMENT, "pipeline must be 0, 1 or 2");
        ako::g_rms_tuning.pipeline = value;
        return AKO_OK;
      }
      if (key == 10) {
        if (value > 32) return fail(AKO_ERR_INVALID_ARGUMENT, "pipelined workgroups per CU above 32");
        ako::g_rms_tuning.pipe_blocks_per_cu = value;
        return AKO_OK;
      }
      if (key == 11) {
        if (value > 2) return fail(AKO_ERR_INVALID_ARGUMENT, "load groups must be 0, 1 or 2");
        ako::g_rms_tuning.load_groups = value;
        return AKO_OK;
      }
      if (key == 12) {
        if (value > 2) return fail(AKO_ERR_INVALID_ARGUMENT, "write-through stores must be 0, 1 or 2");
        ako::g_rms_tuning.write_through = value;
        return AKO_OK;
      }
      break;
    case 1:
      if (key == 1) { ako::g_rope_tuning.tokens_per_block = value; return AKO_OK; }
      if (key == 2) { ako::g_rope_tuning.iters = value; return AKO_OK; }
      if (key == 3) { ako::g_rope_tuning.xcd_chunk = value; return AKO_OK; }
      break;
    case 2:
      if (key == 1) { ako::g_swiglu_tuning.vecs_per_thread = value; return AKO_OK; }
      if (key == 2) { ako::g_swiglu_tuning.xcd_chunk = value; return AKO_OK; }
      break;
    default:
      break;
  }
  return fail(AKO_ERR_INVALID_ARGUMENT, "unknown tuning key op=%d key=%d", op, key);
}

// ---------------------------------------------------------------- RMSNorm --
static int rmsnorm_common(const void* x, const void* r, const void* w, void* y, void* rout,
                          int64_t rows, int64_t hidden, int64_t sx, int64_t sr, int64_t sy,
                          int64_t srout, float eps, int dtype, int w_dtype, void* stream,
                          bool residual) {
  const char* fn = residual ? "ako_rmsnorm_residual_fwd" : "ako_rmsnorm_fwd";
  if (!valid_dtype(dtype)) return fail(AKO_ERR_UNSUPPORTED, "%s: unknown dtype code %d", fn, dtype);
  if (w_dtype != dtype && w_dtype != AKO_DTYPE_F32)
    return fail(AKO_ERR_UNSUPPORTED, "%s: weight dtype %s with input dtype %s (weight must match or be f32)",
                fn, dtype_name(w_dtype), dtype_name(dtype));
  if (rows < 0 || hidden < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative size rows=%lld hidden=%lld", fn, (long long)rows, (long long)hidden);
  if (rows == 0 || hidden == 0) return AKO_OK;
  if (hidden > kMaxInt) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: hidden=%lld exceeds 2^31-1", fn, (long long)hidden);
  if (!x || !w || !y || (residual && (!r || !rout)))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: null pointer argument", fn);
  if (!(eps >= 0.0f)) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: eps must be >= 0", fn);
  if (sx < 0 || sy < 0 || (residual && (sr < 0 || srout < 0)))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative row stride", fn);
  if (rows > 1 && (sy < hidden || (residual && srout < hidden)))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output row stride smaller than hidden (rows would overlap)", fn);
  const int eb = ako::dtype_bytes(dtype);
  const Span sy_span = span_2d(y, rows, hidden, sy, eb);
  const Span sx_span = span_2d(x, rows, hidden, sx, eb);
  const Span w_span = span_2d(w, 1, hidden, hidden, ako::dtype_bytes(w_dtype));
  if (!sy_span.ok || !sx_span.ok ||
      (residual && (!span_2d(r, rows, hidden, sr, eb).ok || !span_2d(rout, rows, hidden, srout, eb).ok)))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: sizes and strides overflow the address space", fn);
  if (overlap(sy_span, sx_span) || overlap(sy_span, w_span))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output y overlaps an input", fn);
  if (residual) {
    const Span sr_span = span_2d(r, rows, hidden, sr, eb);
    const Span so_span = span_2d(rout, rows, hidden, srout, eb);
    if (overlap(sy_span, sr_span) || overlap(so_span, sx_span) || overlap(so_span, sr_span) ||
        overlap(so_span, w_span) || overlap(so_span, sy_span))
      return fail(AKO_ERR_INVALID_ARGUMENT, "%s: residual_out overlaps another buffer", fn);
  }
  bool vec = aligned(x, 16) && aligned(y, 16) && aligned(w, 16) && (sx * eb) % 16 == 0 &&
             (sy * eb) % 16 == 0;
  if (residual) vec = vec && aligned(r, 16) && aligned(rout, 16) && (sr * eb) % 16 == 0 && (srout * eb) % 16 == 0;
  // Rows with a padded stride may be vector-aligned while hidden is not a
  // multiple of the packet; the kernel handles that tail with scalar lanes.
  ako::RmsArgs a{x, r, w, y, rout, rows, hidden, sx, sr, sy, srout, eps, dtype, w_dtype, residual, vec};
  return hip_status(ako::launch_rmsnorm(a, static_cast<hipStream_t>(stream)), fn);
}

int ako_rmsnorm_fwd(const void* x, const void* w, void* y, int64_t rows, int64_t hidden,
                    int64_t x_row_stride, int64_t y_row_stride, float eps, int dtype, int w_dtype,
                    void* stream) {
  return rmsnorm_common(x, nullptr, w, y, nullptr, rows, hidden, x_row_stride, 0, y_row_stride, 0,
                        eps, dtype, w_dtype, stream, false);
}

int ako_rmsnorm_residual_fwd(const void* x, const void* residual, const void* w, void* y,
                             void* residual_out, int64_t rows, int64_t hidden,
                             int64_t x_row_stride, int64_t r_row_stride, int64_t y_row_stride,
                             int64_t rout_row_stride, float eps, int dtype, int w_dtype,
                             void* stream) {
  return rmsnorm_common(x, residual, w, y, residual_out, rows, hidden, x_row_stride, r_row_stride,
                        y_row_stride, rout_row_stride, eps, dtype, w_dtype, stream, true);
}

// ------------------------------------------- RMSNorm over a sharded row --
int ako_rmsnorm_shard_partial_fwd(const void* x, const void* residual, void* residual_out,
                                  float* partial_ss, int64_t rows, int64_t shard,
                                  int64_t x_row_stride, int64_t r_row_stride,
                                  int64_t rout_row_stride, int dtype, void* stream) {
  const char* fn = "ako_rmsnorm_shard_partial_fwd";
  if (!valid_dtype(dtype)) return fail(AKO_ERR_UNSUPPORTED, "%s: unknown dtype code %d", fn, dtype);
  if (rows < 0 || shard < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative size", fn);
  if (rows == 0) return AKO_OK;
  if (shard > kMaxInt) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: shard=%lld exceeds 2^31-1", fn, (long long)shard);
  const bool res = residual != nullptr;
  if ((residual == nullptr) != (residual_out == nullptr))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: residual and residual_out must both be given or both be null", fn);
  if (!partial_ss || (shard > 0 && !x)) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: null pointer argument", fn);
  if (x_row_stride < 0 || (res && (r_row_stride < 0 || rout_row_stride < 0)))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative row stride", fn);
  if (res && rows > 1 && rout_row_stride < shard)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: residual_out row stride smaller than the shard", fn);
  const int eb = ako::dtype_bytes(dtype);
  const Span ps = span_2d(partial_ss, 1, rows, rows, 4);
  const Span xs = span_2d(x, rows, shard, x_row_stride, eb);
  if (!ps.ok || !xs.ok) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: sizes and strides overflow the address space", fn);
  if (shard > 0 && overlap(ps, xs)) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: partial_ss overlaps x", fn);
  bool vec = aligned(x, 16) && (x_row_stride * eb) % 16 == 0;
  if (res) {
    const Span rs = span_2d(residual, rows, shard, r_row_stride, eb);
    const Span os = span_2d(residual_out, rows, shard, rout_row_stride, eb);
    if (!rs.ok || !os.ok) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: sizes and strides overflow the address space", fn);
    if (shard > 0 && (overlap(os, xs) || overlap(os, rs) || overlap(os, ps) || overlap(ps, rs)))
      return fail(AKO_ERR_INVALID_ARGUMENT, "%s: an output overlaps another buffer", fn);
    vec = vec && aligned(residual, 16) && aligned(residual_out, 16) && (r_row_stride * eb) % 16 == 0 &&
          (rout_row_stride * eb) % 16 == 0;
  }
  ako::RmsShardArgs a{};
  a.x = x;
  a.r = residual;
  a.rout = residual_out;
  a.partial = partial_ss;
  a.rows = rows;
  a.shard = shard;
  a.sx = x_row_stride;
  a.sr = r_row_stride;
  a.srout = rout_row_stride;
  a.dtype = dtype;
  a.residual = res;
  a.vector_ok = vec;
  return hip_status(ako::launch_rmsnorm_shard_partial(a, static_cast<hipStream_t>(stream)), fn);
}

int ako_rmsnorm_shard_apply_fwd(const void* s, const void* w, const float* total_ss, void* y,
                                int64_t rows, int64_t shard, int64_t hidden, int64_t s_row_stride,
                                int64_t y_row_stride, float eps, int dtype, int w_dtype,
                                void* stream) {
  const char* fn = "ako_rmsnorm_shard_apply_fwd";
  if (!valid_dtype(dtype)) return fail(AKO_ERR_UNSUPPORTED, "%s: unknown dtype code %d", fn, dtype);
  if (w_dtype != dtype && w_dtype != AKO_DTYPE_F32)
    return fail(AKO_ERR_UNSUPPORTED, "%s: weight dtype %s with input dtype %s (weight must match or be f32)",
                fn, dtype_name(w_dtype), dtype_name(dtype));
  if (rows < 0 || shard < 0 || hidden < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative size", fn);
  if (rows == 0 || shard == 0) return AKO_OK;
  if (shard > hidden) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: shard %lld larger than hidden %lld", fn,
                                  (long long)shard, (long long)hidden);
  if (shard > kMaxInt) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: shard=%lld exceeds 2^31-1", fn, (long long)shard);
  if (!s || !w || !total_ss || !y) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: null pointer argument", fn);
  if (!(eps >= 0.0f)) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: eps must be >= 0", fn);
  if (s_row_stride < 0 || y_row_stride < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative row stride", fn);
  if (rows > 1 && y_row_stride < shard)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output row stride smaller than the shard", fn);
  const int eb = ako::dtype_bytes(dtype);
  const Span ss = span_2d(s, rows, shard, s_row_stride, eb);
  const Span ys = span_2d(y, rows, shard, y_row_stride, eb);
  const Span ws = span_2d(w, 1, shard, shard, ako::dtype_bytes(w_dtype));
  const Span ts = span_2d(total_ss, 1, rows, rows, 4);
  if (!ss.ok || !ys.ok || !ws.ok || !ts.ok)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: sizes and strides overflow the address space", fn);
  if (overlap(ys, ss) || overlap(ys, ws) || overlap(ys, ts))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output y overlaps an input", fn);
  const bool vec = aligned(s, 16) && aligned(y, 16) && aligned(w, 16) && (s_row_stride * eb) % 16 == 0 &&
                   (y_row_stride * eb) % 16 == 0;
  ako::RmsShardArgs a{};
  a.x = s;
  a.w = w;
  a.total = total_ss;
  a.y = y;
  a.rows = rows;
  a.shard = shard;
  a.hidden = hidden;
  a.sx = s_row_stride;
  a.sy = y_row_stride;
  a.eps = eps;
  a.dtype = dtype;
  a.w_dtype = w_dtype;
  a.vector_ok = vec;
  return hip_status(ako::launch_rmsnorm_shard_apply(a, static_cast<hipStream_t>(stream)), fn);
}

// ------------------------------------------------------------------- RoPE --
extern "C++" {  // C++ helpers inside the C-linkage block
namespace {

struct RopeTensorIn {
  const void* x;
  void* y;
  int64_t heads;
  const int64_t* xs;  // strides b, s, h
  const int64_t* ys;  // strides b, s (cache tensors: slot), h
  bool at_pos;        // output rows are cache slots (*pos + s), cache_len of them
};

// Byte span of a [n0, n1, n2, head_dim] view with the given element strides
// (last dimension contiguous): up to the last element + 1.
Span span_4d(const void* p, int64_t n0, int64_t n1, int64_t n2, int64_t d, const int64_t* st, int elem) {
  const __int128 last = static_cast<__int128>(n0 - 1) * st[0] + static_cast<__int128>(n1 - 1) * st[1] +
                        static_cast<__int128>(n2 - 1) * st[2] + d;
  return span_bytes(p, last * elem);
}

// True when distinct (i0, i1, i2, e) of a [n0, n1, n2, head_dim] view address
// distinct elements: taken in order of increasing stride, every dimension of
// more than one index must step past everything the smaller ones span. Any
// nesting order passes (heads-major cache slabs as well as token-major views).
bool distinct_rows(int64_t n0, int64_t n1, int64_t n2, int64_t head_dim, const int64_t* st) {
  struct Dim { int64_t stride, count; } dims[3] = {{st[0], n0}, {st[1], n1}, {st[2], n2}};
  for (int i = 0; i < 3; ++i)
    for (int j = i + 1; j < 3; ++j)
      if (dims[j].stride < dims[i].stride) std::swap(dims[i], dims[j]);
  __int128 reach = head_dim;
  for (const Dim& d : dims) {
    if (d.count <= 1) continue;
    if (d.stride < reach) return false;
    reach += static_cast<__int128>(d.stride) * (d.count - 1);
  }
  return true;
}

// Cache mode: pos != nullptr. Tensors with at_pos write rows 0..cache_len-1
// (selected on the device by *pos + s); the tables must hold table_rows >=
// cache_len rows. Tensor index 2 is copied, not rotated.
int rope_common(const char* fn, const RopeTensorIn* ts, int nt, const void* cos, const void* sin,
                int64_t batch, int64_t seq, int64_t head_dim, int64_t st, int dtype,
                int table_dtype, int style, void* stream, const int64_t* pos = nullptr,
                int64_t cache_len = 0, int64_t table_rows = 0) {
  if (!valid_dtype(dtype) || !valid_dtype(table_dtype))
    return fail(AKO_ERR_UNSUPPORTED, "%s: unknown dtype code (x %d, table %d)", fn, dtype, table_dtype);
  if (style != AKO_ROPE_NEOX && style != AKO_ROPE_INTERLEAVED)
    return fail(AKO_ERR_UNSUPPORTED, "%s: unknown RoPE style %d", fn, style);
  if (batch < 0 || seq < 0 || head_dim < 0)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative size", fn);
  if (head_dim % 2 != 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: head_dim must be even, got %lld", fn, (long long)head_dim);
  const bool cache = pos != nullptr;
  if (cache && (cache_len <= 0 || cache_len > kMaxInt))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: cache_len must be in [1, 2^31-1], got %lld", fn, (long long)cache_len);
  if (cache && table_rows < cache_len)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: the tables hold %lld rows, fewer than cache_len %lld", fn,
                (long long)table_rows, (long long)cache_len);
  int64_t total_heads = 0;
  for (int i = 0; i < nt; ++i) {
    if (ts[i].heads < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative head count", fn);
    total_heads += ts[i].heads;
  }
  if (batch == 0 || seq == 0 || head_dim == 0 || total_heads == 0) return AKO_OK;
  if (head_dim > kMaxInt) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: head_dim too large", fn);
  if (batch > kMaxInt / seq || total_heads > kMaxInt)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: batch*seq and the head count must stay below 2^31", fn);
  if (!cos || !sin) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: null table pointer", fn);
  const int64_t tab_rows = cache ? cache_len : seq;  // rows the kernel may read
  if (st < head_dim / 2 && tab_rows > 1) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: table row stride %lld < head_dim/2", fn, (long long)st);
  const int eb = ako::dtype_bytes(dtype);
  const int tb = ako::dtype_bytes(table_dtype);
  const Span cos_span = span_2d(cos, tab_rows, head_dim / 2, st, tb);
  const Span sin_span = span_2d(sin, tab_rows, head_dim / 2, st, tb);
  if (!cos_span.ok || !sin_span.ok)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: table sizes and strides overflow the address space", fn);
  Span out_spans[3], in_spans[3];
  for (int i = 0; i < nt; ++i) {
    const RopeTensorIn& t = ts[i];
    if (t.heads == 0) continue;
    if (!t.x || !t.y || !t.xs || !t.ys) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: null tensor pointer", fn);
    for (int k = 0; k < 3; ++k)
      if (t.xs[k] < 0 || t.ys[k] < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative stride", fn);
    const int64_t out_rows = t.at_pos ? cache_len : seq;
    // Distinct output elements must not alias.
    if (!distinct_rows(batch, out_rows, t.heads, head_dim, t.ys))
      return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output strides make rows overlap", fn);
    in_spans[i] = span_4d(t.x, batch, seq, t.heads, head_dim, t.xs, eb);
    out_spans[i] = span_4d(t.y, batch, out_rows, t.heads, head_dim, t.ys, eb);
    if (!in_spans[i].ok || !out_spans[i].ok)
      return fail(AKO_ERR_INVALID_ARGUMENT, "%s: sizes and strides overflow the address space", fn);
  }
  if (cache) {
    const Span pos_span{reinterpret_cast<uintptr_t>(pos), reinterpret_cast<uintptr_t>(pos) + sizeof(int64_t)};
    for (int i = 0; i < nt; ++i)
      if (ts[i].heads != 0 && overlap(out_spans[i], pos_span))
        return fail(AKO_ERR_INVALID_ARGUMENT, "%s: an output overlaps pos", fn);
  }
  for (int i = 0; i < nt; ++i) {
    if (ts[i].heads == 0) continue;
    if (overlap(out_spans[i], cos_span) || overlap(out_spans[i], sin_span))
      return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output overlaps a table", fn);
    for (int k = 0; k < nt; ++k) {
      if (ts[k].heads == 0) continue;
      if (overlap(out_spans[i], in_spans[k]))
        return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output overlaps an input", fn);
      if (k != i && overlap(out_spans[i], out_spans[k]))
        return fail(AKO_ERR_INVALID_ARGUMENT, "%s: two outputs overlap", fn);
    }
  }

  const bool neox = style == AKO_ROPE_NEOX;
  const int64_t E = 16 / eb;
  const int64_t unit = neox ? head_dim / 2 : head_dim;
  const int64_t table_vals = neox ? E : E / 2;  // table values one lane loads
  const int64_t tab_align = std::min<int64_t>(16, table_vals * tb);
  bool vec = unit % E == 0 && unit / E <= 64 && aligned(cos, tab_align) && aligned(sin, tab_align) &&
             (st * tb) % tab_align == 0;
  for (int i = 0; i < nt && vec; ++i) {
    const RopeTensorIn& t = ts[i];
    if (t.heads == 0) continue;
    vec = aligned(t.x, 16) && aligned(t.y, 16);
    for (int k = 0; k < 3 && vec; ++k) vec = t.xs[k] % E == 0 && t.ys[k] % E == 0;
  }

  ako::RopeArgs a{};
  const ako::RopeTensorArgs none{nullptr, nullptr, 0, 0, 0, 0, 0, 0, 0};
  auto conv = [&](const RopeTensorIn& t) {
    if (t.heads == 0) return none;
    return ako::RopeTensorArgs{t.x, t.y, t.heads, t.xs[0], t.xs[1], t.xs[2], t.ys[0], t.ys[1], t.ys[2]};
  };
  a.t0 = conv(ts[0]);
  a.t1 = nt > 1 ? conv(ts[1]) : none;
  a.t2 = nt > 2 ? conv(ts[2]) : none;
  // Without a cache the roles of t0 and t1 are the same; a launch with only
  // the second tensor moves it first. In cache mode the roles differ (t0 is
  // written at s, t1 at the cache slot) and an empty t0 simply has no heads.
  if (!cache && a.t0.heads == 0) { a.t0 = a.t1; a.t1 = none; }
  a.pos = pos;
  a.cache_len = cache ? cache_len : 0;
  a.cos = cos;
  a.sin = sin;
  a.batch = batch;
  a.seq = seq;
  a.head_dim = head_dim;
  a.st = st;
  a.dtype = dtype;
  a.table_dtype = table_dtype;
  a.neox = neox;
  a.vector_ok = vec;
  return hip_status(ako::launch_rope(a, static_cast<hipStream_t>(stream)), fn);
}

}  // namespace
}  // extern "C++"

int ako_rope_fwd(const void* x, const void* cos_table, const void* sin_table, void* y,
                 int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int64_t x_stride_b,
                 int64_t x_stride_s, int64_t x_stride_h, int64_t y_stride_b, int64_t y_stride_s,
                 int64_t y_stride_h, int64_t table_row_stride, int dtype, int table_dtype,
                 int style, void* stream) {
  const int64_t xs[3] = {x_stride_b, x_stride_s, x_stride_h};
  const int64_t ys[3] = {y_stride_b, y_stride_s, y_stride_h};
  const RopeTensorIn t{x, y, heads, xs, ys, false};
  return rope_common("ako_rope_fwd", &t, 1, cos_table, sin_table, batch, seq, head_dim,
                     table_row_stride, dtype, table_dtype, style, stream);
}

int ako_rope_qk_fwd(const void* q, const void* k, const void* cos_table, const void* sin_table,
                    void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t q_heads,
                    int64_t k_heads, int64_t head_dim, const int64_t* q_strides,
                    const int64_t* k_strides, const int64_t* q_out_strides,
                    const int64_t* k_out_strides, int64_t table_row_stride, int dtype,
                    int table_dtype, int style, void* stream) {
  const RopeTensorIn ts[2] = {{q, q_out, q_heads, q_strides, q_out_strides, false},
                              {k, k_out, k_heads, k_strides, k_out_strides, false}};
  return rope_common("ako_rope_qk_fwd", ts, 2, cos_table, sin_table, batch, seq, head_dim,
                     table_row_stride, dtype, table_dtype, style, stream);
}

int ako_rope_qk_cache_fwd(const void* q, const void* k, const void* v, const void* cos_table,
                          const void* sin_table, void* q_out, void* k_cache, void* v_cache,
                          const int64_t* pos, int64_t batch, int64_t seq, int64_t q_heads,
                          int64_t kv_heads, int64_t head_dim, const int64_t* q_strides,
                          const int64_t* k_strides, const int64_t* v_strides,
                          const int64_t* q_out_strides, const int64_t* cache_strides,
                          int64_t cache_len, int64_t table_rows, int64_t table_row_stride,
                          int dtype, int table_dtype, int style, void* stream) {
  const char* fn = "ako_rope_qk_cache_fwd";
  if (!pos) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: null pos pointer", fn);
  if ((v == nullptr) != (v_cache == nullptr))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: v and v_cache must both be given or both be null", fn);
  const int64_t v_heads = v ? kv_heads : 0;
  const RopeTensorIn ts[3] = {{q, q_out, q_heads, q_strides, q_out_strides, false},
                              {k, k_cache, kv_heads, k_strides, cache_strides, true},
                              {v, v_cache, v_heads, v_strides, cache_strides, true}};
  return rope_common(fn, ts, 3, cos_table, sin_table, batch, seq, head_dim, table_row_stride, dtype,
                     table_dtype, style, stream, pos, cache_len, table_rows);
}

// ----------------------------------------------------------------- SwiGLU --
int ako_swiglu_fwd(const void* gate, const void* up, void* y, int64_t rows, int64_t n,
                   int64_t gate_row_stride, int64_t up_row_stride, int64_t y_row_stride,
                   int dtype, void* stream) {
  const char* fn = "ako_swiglu_fwd";
  if (!valid_dtype(dtype)) return fail(AKO_ERR_UNSUPPORTED, "%s: unknown dtype code %d", fn, dtype);
  if (rows < 0 || n < 0) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative size", fn);
  if (rows == 0 || n == 0) return AKO_OK;
  if (n > kMaxInt) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: n=%lld exceeds 2^31-1", fn, (long long)n);
  if (!gate || !up || !y) return fail(AKO_ERR_INVALID_ARGUMENT, "%s: null pointer argument", fn);
  if (gate_row_stride < 0 || up_row_stride < 0 || y_row_stride < 0)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: negative row stride", fn);
  if (rows > 1 && y_row_stride < n)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output row stride smaller than n (rows would overlap)", fn);
  const int eb = ako::dtype_bytes(dtype);
  const Span ys = span_2d(y, rows, n, y_row_stride, eb);
  const Span gs = span_2d(gate, rows, n, gate_row_stride, eb);
  const Span us = span_2d(up, rows, n, up_row_stride, eb);
  if (!ys.ok || !gs.ok || !us.ok)
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: sizes and strides overflow the address space", fn);
  if (overlap(ys, gs) || overlap(ys, us))
    return fail(AKO_ERR_INVALID_ARGUMENT, "%s: output overlaps an input", fn);
  const bool contiguous = rows == 1 || (gate_row_stride == n && up_row_stride == n && y_row_stride == n);
  const bool vec = aligned(gate, 16) && aligned(up, 16) && aligned(y, 16) &&
                   (contiguous || ((gate_row_stride * eb) % 16 == 0 && (up_row_stride * eb) % 16 == 0 &&
                                   (y_row_stride * eb) % 16 == 0));
  ako::SwigluArgs a{gate, up, y, rows, n, gate_row_stride, up_row_stride, y_row_stride, dtype,
                    contiguous, vec};
  return hip_status(ako::launch_swiglu(a, static_cast<hipStream_t>(stream)), fn);
}

}  // extern "C"

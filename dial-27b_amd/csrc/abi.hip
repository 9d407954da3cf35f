// C ABI of the dialq library (include/dialq.h): handle lifetime, argument
// validation with the reference's error messages, buffer staging for host
// pointers, and kernel dispatch.  Nothing here throws across the ABI; every
// failure returns -1 / NULL with a NUL-terminated message.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/dialq.h"
#include "common.hpp"
#include "kernels.hpp"

namespace {

using namespace dialq;

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw Error(buf);
}

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) fail("%s failed: %s", what, hipGetErrorString(e));
}

void write_error(char *error, size_t error_size, const char *msg) {
  if (error && error_size > 0) {
    snprintf(error, error_size, "%s", msg);
  }
}

// Device memory owned by a handle or a call.
struct DevBuf {
  void *p = nullptr;
  size_t n = 0;
  DevBuf() = default;
  explicit DevBuf(size_t bytes) { alloc(bytes); }
  void alloc(size_t bytes) {
    release();
    if (bytes) hip_check(hipMalloc(&p, bytes), "hipMalloc");
    n = bytes;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  ~DevBuf() { release(); }
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
};

// One int of pinned, device-mapped host memory that kernels write with
// system-scope stores and the host reads without synchronising.
struct HostWord {
  int *h = nullptr;  // host address
  int *d = nullptr;  // device address of the same word
  void alloc() {
    hip_check(hipHostMalloc((void **)&h, 64, hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc");
    *h = 0;
    hip_check(hipHostGetDevicePointer((void **)&d, h, 0), "hipHostGetDevicePointer");
  }
  ~HostWord() {
    if (h) (void)hipHostFree(h);
  }
};

// Restores the caller's current device on scope exit.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    hip_check(hipGetDevice(&prev), "hipGetDevice");
    if (prev != dev) hip_check(hipSetDevice(dev), "hipSetDevice");
  }
  ~DeviceGuard() {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && prev >= 0 && cur != prev) (void)hipSetDevice(prev);
  }
};

struct Linear {
  dialq_linear_desc desc{};
  int device = 0;
  int64_t n_strips = 0, k_chunks = 0, nbk = 0;
  DevBuf tiles, aux, row_scale, block_scale;
  DevBuf act_scratch;  // activation codes for native prefill / local q8
  DevBuf gemv_ws;  // stream-K partials of the decode GEMV
  DevBuf gemv_cnt; // per-strip piece counters + work-queue head/exit count (zero between calls)
  DevBuf native_part;  // stream-K partial tiles of the native prefill
  DevBuf native_cnt;   // its per-tile arrival counters (zero between calls)
  DevBuf xstage;       // 16-byte-aligned copy of an x that arrives misaligned
  HostWord gave_up;    // set by a decode launch whose bounded wait gave up
  std::mutex scratch_mu;
  float global = 1.0f;

  WeightView view() const {
    WeightView w;
    w.fmt = desc.format;
    w.N = desc.out_dim;
    w.K = desc.in_dim;
    w.n_strips = n_strips;
    w.k_chunks = k_chunks;
    w.nbk = nbk;
    w.tiles = (const uint8_t *)tiles.p;
    w.aux = (const uint8_t *)aux.p;
    w.row_scale = (const float *)row_scale.p;
    w.block_scale = (const float *)block_scale.p;
    w.global = global;
    return w;
  }
};

const char *format_name(int fmt) {
  switch (fmt) {
    case DIALQ_FORMAT_W8A16: return "W8A16";
    case DIALQ_FORMAT_Q8_0: return "Q8_0";
    case DIALQ_FORMAT_Q4_K: return "Q4_K";
    case DIALQ_FORMAT_Q6_K: return "Q6_K";
    case DIALQ_FORMAT_FP8_ROW: return "FP8";
    case DIALQ_FORMAT_FP8_BLOCK: return "FP8 block";
    case DIALQ_FORMAT_NVFP4: return "NVFP4";
    case DIALQ_FORMAT_MXFP4: return "MXFP4";
  }
  return "unknown";
}

size_t dtype_size(int dt) {
  switch (dt) {
    case DIALQ_F32: return 4;
    case DIALQ_F16:
    case DIALQ_BF16: return 2;
  }
  fail("unsupported dtype %d (expected 0=f32, 1=f16, 2=bf16)", dt);
}

// Raw byte sizes of a format's weight and scale buffers.
void raw_sizes(const dialq_linear_desc &d, size_t &wbytes, size_t &sbytes, size_t &scount) {
  const int64_t N = d.out_dim, K = d.in_dim;
  switch (d.format) {
    case DIALQ_FORMAT_W8A16:
      wbytes = (size_t)(N * K);
      scount = (size_t)N;
      sbytes = scount * (d.scale_dtype == DIALQ_BF16 ? 2 : 4);
      return;
    case DIALQ_FORMAT_Q8_0:
      wbytes = (size_t)(N * (K / 32) * 34);
      sbytes = scount = 0;
      return;
    case DIALQ_FORMAT_Q4_K:
      wbytes = (size_t)(N * (K / 256) * 144);
      sbytes = scount = 0;
      return;
    case DIALQ_FORMAT_Q6_K:
      wbytes = (size_t)(N * (K / 256) * 210);
      sbytes = scount = 0;
      return;
    case DIALQ_FORMAT_FP8_ROW:
      wbytes = (size_t)(N * K);
      scount = (size_t)N;
      sbytes = scount * 4;
      return;
    case DIALQ_FORMAT_FP8_BLOCK:
      wbytes = (size_t)(N * K);
      scount = (size_t)(((N + 127) / 128) * ((K + 127) / 128));
      sbytes = scount * 4;
      return;
    case DIALQ_FORMAT_NVFP4:
      wbytes = (size_t)(N * K / 2);
      scount = (size_t)(N * K / 16);
      sbytes = scount;
      return;
    case DIALQ_FORMAT_MXFP4:
      wbytes = (size_t)(N * K / 2);
      scount = (size_t)(N * K / 32);
      sbytes = scount;
      return;
  }
  fail("unknown weight format %d", d.format);
}

void validate_desc(const dialq_linear_desc *d) {
  if (!d) fail("desc is NULL");
  if (d->out_dim <= 0 || d->in_dim <= 0)
    fail("invalid %s shape [%lld, %lld]", format_name(d->format), (long long)d->out_dim,
         (long long)d->in_dim);
  FormatGeom fg = format_geom(d->format);
  if (fg.chunk == 0) fail("unknown weight format %d", d->format);
  // Messages follow CudaQuantLinear::nvfp4 (cuda_quant.rs:301-303) and
  // decode_nvfp4_values (quant.rs:167-171).
  if (d->format == DIALQ_FORMAT_NVFP4 && d->in_dim % 16 != 0)
    fail("NVFP4 QuantLinear input dimension %lld is not divisible by 16", (long long)d->in_dim);
  if (d->in_dim % fg.k_align != 0)
    fail("%s input dimension %lld is not divisible by %d", format_name(d->format),
         (long long)d->in_dim, fg.k_align);
  if (d->format == DIALQ_FORMAT_W8A16 && d->scale_dtype != DIALQ_F32 && d->scale_dtype != DIALQ_BF16)
    fail("W8A16 scale dtype must be f32 or bf16, got %d", d->scale_dtype);
  if (d->format == DIALQ_FORMAT_NVFP4) {
    float gs = d->global_scale;
    if (!(gs == gs) || gs == 0.0f)
      fail("NVFP4 global scale must contain one non-zero value, got %g", (double)gs);
  }
}

Linear *alloc_linear(const dialq_linear_desc &d, int device) {
  Linear *L = new Linear();
  L->desc = d;
  L->device = device;
  FormatGeom fg = format_geom(d.format);
  L->n_strips = (d.out_dim + 15) / 16;
  L->k_chunks = (d.in_dim + fg.chunk - 1) / fg.chunk;
  L->nbk = (d.in_dim + 127) / 128;
  L->tiles.alloc((size_t)(L->n_strips * L->k_chunks * fg.tile_bytes));
  if (fg.aux_bytes) L->aux.alloc((size_t)(L->n_strips * L->k_chunks * fg.aux_bytes));
  if (d.format == DIALQ_FORMAT_W8A16 || d.format == DIALQ_FORMAT_FP8_ROW)
    L->row_scale.alloc((size_t)(L->n_strips * 16) * sizeof(float));
  if (d.format == DIALQ_FORMAT_FP8_BLOCK)
    L->block_scale.alloc((size_t)(((d.out_dim + 127) / 128) * L->nbk) * sizeof(float));
  if (d.format == DIALQ_FORMAT_NVFP4) {
    L->global = (d.flags & DIALQ_FLAG_GLOBAL_IS_DIVISOR) ? 1.0f / d.global_scale : d.global_scale;
  }
  try {
    L->gemv_cnt.alloc((size_t)(L->n_strips + 2) * sizeof(int));  // strips, queue head, exit count
    hip_check(hipMemset(L->gemv_cnt.p, 0, L->gemv_cnt.n), "hipMemset");
    L->gave_up.alloc();
  } catch (...) {
    delete L;
    throw;
  }
  return L;
}

// Copy `bytes` from a host or device source into a fresh device buffer.
void stage_in(DevBuf &dst, const void *src, size_t bytes, bool host, hipStream_t st) {
  dst.alloc(bytes);
  if (bytes)
    hip_check(hipMemcpyAsync(dst.p, src, bytes, host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice, st),
              "hipMemcpyAsync");
}

template <typename F>
int guarded(char *error, size_t error_size, F &&f) {
  try {
    f();
    if (error && error_size) error[0] = '\0';
    return 0;
  } catch (const std::exception &e) {
    write_error(error, error_size, e.what());
  } catch (...) {
    write_error(error, error_size, "unknown error");
  }
  return -1;
}

// A handle's scratch buffers (GEMV workspace, native prefill codes and
// partials, the aligned copy of x) are owned by the handle (calls on one
// handle are stream-ordered) and grow on demand: after the stream has
// drained, since earlier launches may still use the old buffer, and never
// during stream capture, where the allocation would not be replayed -- a
// capture must follow an eager call of at least the same shape.
void refuse_growth_in_capture(hipStream_t st, const char *what, size_t bytes) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hip_check(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    fail("%s must grow to %zu bytes during stream capture; run one eager call of this shape before capturing", what,
         bytes);
}

void grow(DevBuf &b, size_t bytes, hipStream_t st, const char *what) {
  if (b.n >= bytes) return;
  refuse_growth_in_capture(st, what, bytes);
  hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  b.alloc(bytes);
}

void ensure_scratch(Linear *L, size_t bytes, hipStream_t st) { grow(L->act_scratch, bytes, st, "activation scratch"); }

// Stream-K partials and tile counters of the native prefill.
void ensure_native_scratch(Linear *L, size_t part_bytes, size_t cnt_count, hipStream_t st) {
  const size_t cnt_bytes = cnt_count * sizeof(int);
  if (L->native_part.n >= part_bytes && L->native_cnt.n >= cnt_bytes) return;
  grow(L->native_part, part_bytes, st, "native prefill partials");
  if (L->native_cnt.n < cnt_bytes) {
    grow(L->native_cnt, cnt_bytes, st, "native prefill tile counters");
    hip_check(hipMemsetAsync(L->native_cnt.p, 0, cnt_bytes, st), "hipMemsetAsync");
  }
}

// The scratch one forward call takes, by region, for the kernel it picks.
struct ForwardPlan {
  int path = DIALQ_PATH_AUTO;  // resolved: GEMV, GEMM or GEMM_NATIVE
  int64_t k_pad = 0;           // native: padded K of the activation codes
  size_t gemv_ws = 0;          // decode workspace (stream-K / work-queue partials)
  size_t gemv_cnt = 0;         // decode counters (ints): n_strips + 2
  size_t codes = 0;            // native: activation codes, rounded up to 256 bytes
  size_t xscale = 0;           // native: activation scales
  size_t part = 0;             // native: split-K partial tiles
  size_t ncnt = 0;             // native: split-K tile counters (ints)
  size_t xh = 0;               // Q4_K / Q8_0 GEMM on bf16 x: its f16 copy, then the row scales
};

// Bytes of the f16 copy of a bf16 x (and its row scales) that the GGUF
// (Q4_K, Q8_0) prefill kernel multiplies; 0 where that path does not apply.
size_t kq_f16_stage_bytes(const Linear *L, int x_dtype, int64_t rows, int path) {
  const int fmt = L->desc.format;
  if (path != DIALQ_PATH_GEMM || x_dtype != DIALQ_BF16 ||
      (fmt != DIALQ_FORMAT_Q4_K && fmt != DIALQ_FORMAT_Q8_0 && fmt != DIALQ_FORMAT_Q6_K))
    return 0;
  return (size_t)(rows * L->desc.in_dim * 2 + 255) / 256 * 256 + (size_t)rows * sizeof(float);
}

// Where a call's scratch lives: the handle's own buffers, grown on demand,
// or the allocation-free entry point's static array.  Counters are zero
// before the call and are left zero by the kernels.
struct ForwardBufs {
  float *gemv_ws = nullptr;
  size_t gemv_ws_bytes = 0;
  int *gemv_cnt = nullptr;
  uint8_t *codes = nullptr;
  void *xscale = nullptr;
  float *part = nullptr;
  size_t part_bytes = 0;
  int *ncnt = nullptr;
  size_t ncnt_count = 0;
  uint8_t *xh = nullptr;  // f16 copy of a bf16 x, then its row scales (plan.xh bytes)
};

// A bf16 x of a Q4_K / Q8_0 prefill as f16 rows in range (k_x_f16_rows): returns the
// row scales the GEMM's epilogue multiplies by; `xf` becomes the f16 copy.
const float *stage_kq_f16(const void *x, int64_t rows, int64_t K, uint8_t *buf, const void *&xf, hipStream_t st) {
  uint16_t *xh = (uint16_t *)buf;
  float *rs = (float *)(buf + (size_t)(rows * K * 2 + 255) / 256 * 256);
  hip_check(launch_x_f16_rows(x, rows, K, xh, rs, st), "bf16 -> f16 activation rows");
  xf = xh;
  return rs;
}

WeightView forward_view(const Linear *L, bool swiglu) {
  WeightView w = L->view();
  if (swiglu) w.pair = L->desc.out_dim / 32;  // gate / up halves of out_dim / 2 rows, 16 rows per strip
  return w;
}

// stage_f16: a Q4_K / Q8_0 GEMM on bf16 x runs the f16 kernel on an f16 copy of x
// (false: the bf16 hi / lo kernel, no copy).
// tail: split the tiles of a partial last round of workgroups (more
// scratch; false where the allocation-free entry point has no room).
ForwardPlan plan_forward(const Linear *L, const WeightView &w, int x_dtype, int64_t rows, int path,
                         bool stage_f16 = true, bool tail = true) {
  const int fmt = L->desc.format;
  ForwardPlan pl;
  if (path == DIALQ_PATH_AUTO) {
    // the decode kernel re-streams the weight for every 16 rows; past one
    // pass the GEMM (32-row tiles split along K where its tiles are few) is
    // faster: 17408x5120 W8A16 at M = 24 36.5 against 71 us, at M = 64 45.5
    // against 163
    if (rows <= 16) path = DIALQ_PATH_GEMV;
    else if ((fmt == DIALQ_FORMAT_FP8_BLOCK || fmt == DIALQ_FORMAT_MXFP4) &&
             !(L->desc.flags & DIALQ_FLAG_WEIGHT_ONLY_PREFILL))
      path = DIALQ_PATH_GEMM_NATIVE;
    else path = DIALQ_PATH_GEMM;
  }
  pl.path = path;
  // every kernel addresses the resident tiles with 32-bit buffer offsets and
  // marks masked loads with an offset of 2^31, past any weight below 2 GiB
  if (L->tiles.n >= ((size_t)1 << 31))
    fail("%s kernel addresses weights with 32-bit offsets: %zu resident bytes exceed 2 GiB; split the "
         "output dimension", path == DIALQ_PATH_GEMV ? "decode" : "prefill", L->tiles.n);
  if (path == DIALQ_PATH_GEMV) {
    pl.gemv_ws = gemv_workspace_bytes(w, x_dtype, rows);
    pl.gemv_cnt = (size_t)(L->n_strips + 2);
  } else if (path == DIALQ_PATH_GEMM_NATIVE) {
    if (fmt != DIALQ_FORMAT_FP8_BLOCK && fmt != DIALQ_FORMAT_MXFP4)
      fail("native fp8/fp4 prefill needs an FP8 block or MXFP4 weight, got %s", format_name(fmt));
    pl.k_pad = w.k_chunks * 128;
    const size_t codes = fmt == DIALQ_FORMAT_FP8_BLOCK ? (size_t)(rows * pl.k_pad) : (size_t)(rows * pl.k_pad / 2);
    pl.codes = (codes + 255) / 256 * 256;
    pl.xscale = fmt == DIALQ_FORMAT_FP8_BLOCK ? (size_t)rows * sizeof(float) : (size_t)(rows * pl.k_pad / 32);
    native_workspace(rows, w, pl.part, pl.ncnt, tail);
  } else if (path == DIALQ_PATH_GEMM) {
    if (stage_f16) pl.xh = kq_f16_stage_bytes(L, x_dtype, rows, path);
    // split-K partials of few-tile launches (the f16 kernel's tiling when x is staged as f16)
    gemm_workspace(rows, w, pl.xh ? DIALQ_F16 : x_dtype, pl.part, pl.ncnt, tail);
  } else {
    fail("unknown path %d", path);
  }
  return pl;
}

void launch_forward(const Linear *L, const WeightView &w, const ForwardPlan &pl, const ForwardBufs &b, const void *x,
                    int x_dtype, int64_t rows, void *y, int y_dtype, hipStream_t st) {
  if (pl.path == DIALQ_PATH_GEMV) {
    hip_check(launch_gemv(w, x, x_dtype, rows, y, y_dtype, b.gemv_ws, b.gemv_ws_bytes, b.gemv_cnt, L->gave_up.d, st),
              "GEMV launch");
  } else if (pl.path == DIALQ_PATH_GEMM) {
    const void *xf = x;
    const float *yrow = b.xh ? stage_kq_f16(x, rows, w.K, b.xh, xf, st) : nullptr;
    hip_check(launch_gemm(w, xf, b.xh ? DIALQ_F16 : x_dtype, rows, y, y_dtype, b.part, b.part_bytes, b.ncnt,
                          b.ncnt_count, st, yrow),
              "GEMM launch");
  } else {
    if (L->desc.format == DIALQ_FORMAT_FP8_BLOCK)
      hip_check(launch_act_fp8(x, x_dtype, rows, w.K, pl.k_pad, b.codes, (float *)b.xscale, st),
                "activation quantizer");
    else
      hip_check(launch_act_mxfp4(x, x_dtype, rows, w.K, pl.k_pad, b.codes, (uint8_t *)b.xscale, st),
                "activation quantizer");
    hip_check(launch_gemm_native(w, b.codes, b.xscale, rows, pl.k_pad, y, y_dtype, b.part, b.part_bytes, b.ncnt,
                                 b.ncnt_count, st),
              "native GEMM launch");
  }
}

// Forward of the weight view `w` of handle L (its own view, or a member's
// view into a concatenated output) with the handle's own scratch, grown on
// demand.
void run_forward(Linear *L, const WeightView &w, const void *x, int x_dtype, int64_t rows, void *y, int y_dtype,
                 int path, hipStream_t st) {
  const ForwardPlan pl = plan_forward(L, w, x_dtype, rows, path);
  std::lock_guard<std::mutex> lock(L->scratch_mu);
  ForwardBufs b;
  if (pl.path == DIALQ_PATH_GEMV) {
    grow(L->gemv_ws, pl.gemv_ws, st, "decode GEMV workspace");
    b.gemv_ws = (float *)L->gemv_ws.p;
    b.gemv_ws_bytes = L->gemv_ws.n;
    b.gemv_cnt = (int *)L->gemv_cnt.p;
  } else {
    if (pl.path == DIALQ_PATH_GEMM_NATIVE) {
      ensure_scratch(L, pl.codes + pl.xscale, st);
      b.codes = (uint8_t *)L->act_scratch.p;
      b.xscale = b.codes + pl.codes;
    } else if (pl.xh) {
      ensure_scratch(L, pl.xh, st);
      b.xh = (uint8_t *)L->act_scratch.p;
    }
    // split-K partials and tile counters (native prefill, or a GEMM of few tiles)
    ensure_native_scratch(L, pl.part, pl.ncnt, st);
    b.part = (float *)L->native_part.p;
    b.part_bytes = L->native_part.n;
    b.ncnt = (int *)L->native_cnt.p;
    b.ncnt_count = L->native_cnt.n / sizeof(int);
  }
  launch_forward(L, w, pl, b, x, x_dtype, rows, y, y_dtype, st);
}

// A decode launch on this handle whose work-queue wait gave up (it wrote
// an incomplete output and may have left the queue counters non-zero) is
// reported by the next forward on the handle, which resets the counters.
void check_gave_up(Linear *L, hipStream_t st) {
  if (!__atomic_load_n(L->gave_up.h, __ATOMIC_ACQUIRE)) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hip_check(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    fail("a previous decode launch on this handle gave up waiting for its work queue and left an incomplete "
         "output; the handle cannot be reset during stream capture");
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");  // the launch that gave up has ended
  hip_check(hipMemset(L->gemv_cnt.p, 0, L->gemv_cnt.n), "hipMemset");
  __atomic_store_n(L->gave_up.h, 0, __ATOMIC_RELEASE);
  fail("a previous decode launch on this handle gave up waiting for its work queue after %d polls without "
       "progress; that call's output is incomplete.  The handle's queue counters are reset and the next call "
       "runs normally", gemv_wait_limit());
}

void forward_impl(Linear *L, const void *x, int32_t x_dtype, int64_t rows, void *y, int32_t y_dtype,
                  int32_t path, void *stream, int device_io, bool local_q8, bool swiglu = false) {
  if (!L) fail("linear handle is NULL");
  if (rows < 0) fail("rows must be >= 0, got %lld", (long long)rows);
  size_t xs = dtype_size(x_dtype), ys = dtype_size(y_dtype);
  if (swiglu && L->desc.out_dim % 128 != 0)
    fail("SwiGLU forward needs a fused gate_up weight whose out_dim (%lld) is a multiple of 128: gate and up "
         "halves of a multiple of 64 rows", (long long)L->desc.out_dim);
  if (rows == 0) return;
  if (!x || !y) fail("x and y must not be NULL");
  DeviceGuard dg(L->device);
  hipStream_t st = (hipStream_t)stream;
  check_gave_up(L, st);
  const int64_t N = swiglu ? L->desc.out_dim / 2 : L->desc.out_dim, K = L->desc.in_dim;
  size_t xbytes = (size_t)(rows * K) * xs, ybytes = (size_t)(rows * N) * ys;
  DevBuf dx, dy;
  const void *xp = x;
  void *yp = y;
  if (!device_io) {
    stage_in(dx, x, xbytes, true, st);
    dy.alloc(ybytes);
    xp = dx.p;
    yp = dy.p;
  } else if (((uintptr_t)x) & 15u) {
    // The kernels read x with 16-byte buffer loads and LDS DMA from a
    // 16-byte-aligned base.  A view at any other offset (a candle narrow /
    // start_offset, worker_w8a16.rs:419) is copied once into the handle's
    // aligned staging buffer, on the same stream.
    std::lock_guard<std::mutex> lock(L->scratch_mu);
    grow(L->xstage, xbytes, st, "aligned copy of a misaligned x");
    hip_check(hipMemcpyAsync(L->xstage.p, x, xbytes, hipMemcpyDeviceToDevice, st), "hipMemcpyAsync");
    xp = L->xstage.p;
  }
  if (((uintptr_t)yp) % ys) fail("y must be aligned to its element size (%zu bytes)", ys);
  if (local_q8) {
    if (L->desc.format != DIALQ_FORMAT_W8A16 || L->desc.scale_dtype != DIALQ_F32)
      fail("local q8 linear needs a W8A16 weight with f32 scales");
    if (rows != 1) fail("local q8 linear expects decode [1, 1, %lld], got %lld rows", (long long)K, (long long)rows);
    std::lock_guard<std::mutex> lock(L->scratch_mu);
    int64_t k_pad = L->k_chunks * 64;
    ensure_scratch(L, (size_t)((k_pad + 255) / 256 * 256 + 256), st);
    hip_check(launch_local_q8(L->view(), xp, x_dtype, yp, y_dtype, L->act_scratch.p, st), "local q8 launch");
  } else {
    run_forward(L, forward_view(L, swiglu), xp, x_dtype, rows, yp, y_dtype, path, st);
  }
  if (!device_io) {
    hip_check(hipMemcpyAsync(y, yp, ybytes, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  }
}

// ---- grouped forward ---------------------------------------------------------
// y = cat([x W_0^T, ..., x W_{n-1}^T], -1) for handles that share x: the
// decode path runs the strips of up to four same-format members in one
// launch (one workgroup per strip, x staged once per workgroup as in a
// single forward); the prefill paths run the column tiles of up to four
// same-format members in one GEMM launch (W8A16, FP8_ROW, Q4_K and Q8_0 with
// bf16 / f16 x; FP8_BLOCK and MXFP4 native on x quantized once); every other case
// runs one launch per member, each writing its columns of the concatenated
// output.
constexpr int kGroupMax = 4;

// One prefill launch over members Ls[0..n) (one format and K, resolved path
// GEMM or GEMM_NATIVE), with Ls[0]'s scratch: false, launching nothing,
// where no grouped kernel applies.
bool run_prefill_group(Linear *const *Ls, const WeightView *ws, void *const *ys, int n, const void *x, int x_dtype,
                       int64_t rows, int y_dtype, int path, hipStream_t st) {
  Linear *L = Ls[0];
  size_t part = 0, ncnt = 0;
  if (path == DIALQ_PATH_GEMM) {
    const size_t xh = kq_f16_stage_bytes(L, x_dtype, rows, path);  // bf16 x of a Q4_K / Q8_0 group: f16 once
    const int kx = xh ? DIALQ_F16 : x_dtype;
    if (!gemm_group_workspace(rows, ws, n, kx, part, ncnt)) return false;
    std::lock_guard<std::mutex> lock(L->scratch_mu);
    ensure_native_scratch(L, part, ncnt, st);
    const void *xf = x;
    const float *yrow = nullptr;
    if (xh) {
      ensure_scratch(L, xh, st);
      yrow = stage_kq_f16(x, rows, ws[0].K, (uint8_t *)L->act_scratch.p, xf, st);
    }
    const hipError_t r = launch_gemm_group(ws, ys, n, xf, kx, rows, y_dtype, (float *)L->native_part.p,
                                           L->native_part.n, (int *)L->native_cnt.p, L->native_cnt.n / sizeof(int), st,
                                           yrow);
    if (r == hipErrorNotSupported) return false;
    hip_check(r, "grouped GEMM launch");
    return true;
  }
  if (!native_group_workspace(rows, ws, n, part, ncnt)) return false;
  const ForwardPlan pl = plan_forward(L, ws[0], x_dtype, rows, path);  // activation codes, scales, k_pad
  std::lock_guard<std::mutex> lock(L->scratch_mu);
  ensure_scratch(L, pl.codes + pl.xscale, st);
  ensure_native_scratch(L, part, ncnt, st);
  uint8_t *codes = (uint8_t *)L->act_scratch.p;
  void *xscale = codes + pl.codes;
  if (L->desc.format == DIALQ_FORMAT_FP8_BLOCK)
    hip_check(launch_act_fp8(x, x_dtype, rows, ws[0].K, pl.k_pad, codes, (float *)xscale, st), "activation quantizer");
  else
    hip_check(launch_act_mxfp4(x, x_dtype, rows, ws[0].K, pl.k_pad, codes, (uint8_t *)xscale, st),
              "activation quantizer");
  hip_check(launch_gemm_native_group(ws, ys, n, codes, xscale, rows, pl.k_pad, y_dtype, (float *)L->native_part.p,
                                     L->native_part.n, (int *)L->native_cnt.p, L->native_cnt.n / sizeof(int), st),
            "grouped native GEMM launch");
  return true;
}

void forward_group_impl(Linear *const *Ls, int32_t n, const void *x, int32_t x_dtype, int64_t rows, void *y,
                        int32_t y_dtype, int32_t path, void *stream, int device_io) {
  if (!Ls || n < 1) fail("a grouped forward needs at least one handle, got %d", (int)n);
  for (int j = 0; j < n; ++j) {
    if (!Ls[j]) fail("linear handle %d of the group is NULL", j);
    for (int i = 0; i < j; ++i)  // members own their scratch; one handle twice would share it
      if (Ls[i] == Ls[j]) fail("grouped forward: handle %d is the same handle as %d", j, i);
  }
  const int64_t K = Ls[0]->desc.in_dim;
  int64_t ntot = 0;
  for (int j = 0; j < n; ++j) {
    if (Ls[j]->desc.in_dim != K)
      fail("grouped forward: handle %d has in_dim %lld, handle 0 has %lld (the members share x)", j,
           (long long)Ls[j]->desc.in_dim, (long long)K);
    if (Ls[j]->device != Ls[0]->device)
      fail("grouped forward: handle %d lives on device %d, handle 0 on %d", j, Ls[j]->device, Ls[0]->device);
    ntot += Ls[j]->desc.out_dim;
  }
  if (rows < 0) fail("rows must be >= 0, got %lld", (long long)rows);
  const size_t xs = dtype_size(x_dtype), ys = dtype_size(y_dtype);
  if (rows == 0) return;
  if (!x || !y) fail("x and y must not be NULL");
  DeviceGuard dg(Ls[0]->device);
  hipStream_t st = (hipStream_t)stream;
  for (int j = 0; j < n; ++j) check_gave_up(Ls[j], st);
  const size_t xbytes = (size_t)(rows * K) * xs, ybytes = (size_t)(rows * ntot) * ys;
  DevBuf dx, dy;
  const void *xp = x;
  void *yp = y;
  if (!device_io) {
    stage_in(dx, x, xbytes, true, st);
    dy.alloc(ybytes);
    xp = dx.p;
    yp = dy.p;
  } else {
    if (((uintptr_t)yp) % ys) fail("y must be aligned to its element size (%zu bytes)", ys);
    if (((uintptr_t)x) & 15u) {  // staged once, in the first member's buffer
      std::lock_guard<std::mutex> lock(Ls[0]->scratch_mu);
      grow(Ls[0]->xstage, xbytes, st, "aligned copy of a misaligned x");
      hip_check(hipMemcpyAsync(Ls[0]->xstage.p, x, xbytes, hipMemcpyDeviceToDevice, st), "hipMemcpyAsync");
      xp = Ls[0]->xstage.p;
    }
  }
  std::vector<WeightView> views((size_t)n);
  std::vector<void *> outs((size_t)n);
  std::vector<int> paths((size_t)n);
  int64_t off = 0;
  for (int j = 0; j < n; ++j) {
    views[j] = forward_view(Ls[j], false);
    views[j].ldy = ntot;
    outs[j] = (uint8_t *)yp + (size_t)off * ys;
    off += Ls[j]->desc.out_dim;
    paths[j] = plan_forward(Ls[j], views[j], x_dtype, rows, path).path;
  }
  std::vector<bool> done((size_t)n, false);
  // runs of up to four consecutive decode members of one format: one launch
  for (int j = 0; j < n;) {
    int e = j + 1;
    while (e < n && e - j < kGroupMax && paths[e] == DIALQ_PATH_GEMV && paths[j] == DIALQ_PATH_GEMV &&
           Ls[e]->desc.format == Ls[j]->desc.format)
      ++e;
    if (e - j >= 2) {
      for (int i = j; i < e; ++i)
        if (Ls[i]->tiles.n >= ((size_t)1 << 31)) fail("decode kernel addresses weights with 32-bit offsets");
      const hipError_t r = launch_gemv_group(&views[j], &outs[j], e - j, xp, x_dtype, rows, y_dtype, st);
      if (r == hipSuccess)
        for (int i = j; i < e; ++i) done[i] = true;
      else if (r != hipErrorNotSupported)
        hip_check(r, "grouped GEMV launch");
    }
    j = e;
  }
  // runs of up to four consecutive prefill members of one format and path:
  // one GEMM launch over all their column tiles (native: on x quantized once)
  for (int j = 0; j < n;) {
    if (paths[j] != DIALQ_PATH_GEMM && paths[j] != DIALQ_PATH_GEMM_NATIVE) {
      ++j;
      continue;
    }
    int e = j + 1;
    while (e < n && e - j < kGroupMax && paths[e] == paths[j] && Ls[e]->desc.format == Ls[j]->desc.format) ++e;
    if (e - j >= 2 && run_prefill_group(&Ls[j], &views[j], &outs[j], e - j, xp, x_dtype, rows, y_dtype, paths[j], st))
      for (int i = j; i < e; ++i) done[i] = true;
    j = e;
  }
  for (int j = 0; j < n; ++j)
    if (!done[j]) run_forward(Ls[j], views[j], xp, x_dtype, rows, outs[j], y_dtype, path, st);
  if (!device_io) {
    hip_check(hipMemcpyAsync(y, yp, ybytes, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  }
}

// ---- allocation-free forward ------------------------------------------------
// dialq_linear_forward_noalloc takes its scratch from this file-scope
// device array instead of the handle's grown buffers: callers that cannot
// allocate (code under graph capture, tight serving loops) get the same
// kernels with no hipMalloc / hipFree on the call path.  Every device that
// runs the library holds its own copy until the process ends.  Layout:
//   [0, kNoAllocCntBytes)   counters (decode GEMV per-strip / queue counters,
//                           or native split-K tile counters); zero between
//                           calls: zero at load, cleared once per device at
//                           set-up, and left zero by every call that ends
//                           normally (the kernels re-arm them)
//   [kNoAllocCntBytes, ..)  the call's workspace regions, then the aligned
//                           copy of a misaligned x
// Calls on one device share the array: calls that overlap in time on one
// device (different streams, or concurrent host threads) race.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
constexpr size_t kNoAllocCntBytes = 65536;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

__global__ void k_zero_words(uint32_t *p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

std::mutex g_noalloc_mu;
std::vector<uint8_t *> g_noalloc_ptr;  // per device: the array's device address (null until set up)

// The array's address on the current device `dev`, looked up once per
// device (hipGetSymbolAddress with that device current); the counter region
// is cleared on that first use with a fill kernel on `st`.
uint8_t *noalloc_scratch(int dev, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if ((int)g_noalloc_ptr.size() <= dev) g_noalloc_ptr.resize((size_t)dev + 1, nullptr);
  if (!g_noalloc_ptr[dev]) {
    void *ptr = nullptr;
    hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    k_zero_words<<<16, 256, 0, st>>>((uint32_t *)ptr, kNoAllocCntBytes / 4);
    hip_check(hipGetLastError(), "scratch counter clear");
    g_noalloc_ptr[dev] = (uint8_t *)ptr;
  }
  return g_noalloc_ptr[dev];
}

void forward_noalloc_impl(Linear *L, const void *x, int32_t x_dtype, int64_t rows, void *y, int32_t y_dtype,
                          int32_t path, void *stream) {
  if (!L) fail("linear handle is NULL");
  if (rows < 0) fail("rows must be >= 0, got %lld", (long long)rows);
  const size_t xs = dtype_size(x_dtype), ys = dtype_size(y_dtype);
  if (rows == 0) return;
  if (!x || !y) fail("x and y must not be NULL");
  if (((uintptr_t)y) % ys) fail("y must be aligned to its element size (%zu bytes)", ys);
  DeviceGuard dg(L->device);
  hipStream_t st = (hipStream_t)stream;
  uint8_t *base = noalloc_scratch(L->device, st);
  if (__atomic_load_n(L->gave_up.h, __ATOMIC_ACQUIRE)) {
    // a decode launch on this handle gave up: its counters may be left set
    // in the shared array as well as the handle's
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hip_check(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
    if (cs == hipStreamCaptureStatusNone) {
      hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
      k_zero_words<<<16, 256, 0, st>>>((uint32_t *)base, kNoAllocCntBytes / 4);
      hip_check(hipGetLastError(), "scratch counter clear");
    }
    check_gave_up(L, st);
  }
  const int64_t K = L->desc.in_dim;
  const WeightView w = forward_view(L, false);
  auto up = [](size_t v) { return (v + 255) / 256 * 256; };
  const size_t xbytes = (size_t)(rows * K) * xs;
  const bool stage_x = ((uintptr_t)x) & 15u;
  ForwardPlan pl = plan_forward(L, w, x_dtype, rows, path);
  auto fits = [&](const ForwardPlan &q) {
    return kNoAllocCntBytes + up(q.gemv_ws) + up(q.codes + q.xscale) + up(q.part) + up(q.xh) +
               (stage_x ? up(xbytes) : 0) <= kNoAllocScratchBytes;
  };
  // the tail split's partials first give way (the launch then keeps the
  // last round's tiles whole), then a Q4_K / Q8_0 prefill on bf16 x whose
  // f16 copy does not fit runs the bf16 hi / lo kernel on x as it is
  if (!fits(pl)) pl = plan_forward(L, w, x_dtype, rows, path, true, false);
  if (pl.xh && !fits(pl)) pl = plan_forward(L, w, x_dtype, rows, path, false, false);
  const size_t cnt_ints = pl.path == DIALQ_PATH_GEMV ? pl.gemv_cnt : pl.ncnt;
  if (cnt_ints * sizeof(int) > kNoAllocCntBytes)
    fail("dialq_linear_forward_noalloc: this %s weight needs %zu counters; its scratch holds %zu (out_dim up to "
         "%zu rows for the decode path)", format_name(L->desc.format), cnt_ints, kNoAllocCntBytes / sizeof(int),
         (kNoAllocCntBytes / sizeof(int) - 2) * 16);
  // regions after the counters, 256-byte aligned
  size_t off = kNoAllocCntBytes;
  ForwardBufs b;
  if (pl.path == DIALQ_PATH_GEMV) {
    b.gemv_cnt = (int *)base;
    b.gemv_ws = pl.gemv_ws ? (float *)(base + off) : nullptr;
    b.gemv_ws_bytes = pl.gemv_ws;
    off += up(pl.gemv_ws);
  } else {
    if (pl.path == DIALQ_PATH_GEMM_NATIVE) {
      b.codes = base + off;
      b.xscale = base + off + pl.codes;
      off += up(pl.codes + pl.xscale);
    }
    b.part = pl.part ? (float *)(base + off) : nullptr;
    b.part_bytes = pl.part;
    off += up(pl.part);
    b.ncnt = pl.ncnt ? (int *)base : nullptr;
    b.ncnt_count = pl.ncnt;
    if (pl.xh) {
      b.xh = base + off;
      off += up(pl.xh);
    }
  }
  const void *xp = x;
  const size_t need = off + (stage_x ? up(xbytes) : 0);
  if (need > kNoAllocScratchBytes)
    fail("dialq_linear_forward_noalloc: %lld rows of this %s [%lld, %lld] weight need %zu bytes of scratch; the "
         "allocation-free entry point has %zu (use dialq_linear_forward, or fewer rows per call)",
         (long long)rows, format_name(L->desc.format), (long long)L->desc.out_dim, (long long)K, need,
         kNoAllocScratchBytes);
  if (stage_x) {
    hip_check(hipMemcpyAsync(base + off, x, xbytes, hipMemcpyDeviceToDevice, st), "hipMemcpyAsync");
    xp = base + off;
  }
  launch_forward(L, w, pl, b, xp, x_dtype, rows, y, y_dtype, st);
}

}  // namespace

extern "C" {

uint32_t dialq_abi_version(void) { return DIALQ_ABI_VERSION; }

void *dialq_linear_create(const dialq_linear_desc *desc, const void *weight, size_t weight_bytes,
                          const void *scales, size_t scale_bytes, int device, int host_io,
                          void *stream, char *error, size_t error_size) {
  Linear *out = nullptr;
  guarded(error, error_size, [&] {
    validate_desc(desc);
    const dialq_linear_desc &d = *desc;
    size_t wexp, sexp, scount;
    raw_sizes(d, wexp, sexp, scount);
    // Length checks and messages of CudaQuantLinear::nvfp4 / ::fp8
    // (cuda_quant.rs:304-309, 339-344).
    if (d.format == DIALQ_FORMAT_NVFP4) {
      if (weight_bytes != wexp) fail("invalid NVFP4 packed weight length %zu", weight_bytes);
      if (scale_bytes != sexp) fail("invalid NVFP4 scale length %zu", scale_bytes);
    } else if (d.format == DIALQ_FORMAT_FP8_ROW) {
      if (weight_bytes != wexp) fail("invalid FP8 weight length %zu", weight_bytes);
      if (scale_bytes != sexp && scale_bytes != 4) fail("invalid FP8 scale length %zu", scale_bytes / 4);
      scount = scale_bytes / 4;
    } else {
      if (weight_bytes != wexp)
        fail("invalid %s weight length %zu, expected %zu", format_name(d.format), weight_bytes, wexp);
      if (scale_bytes != sexp)
        fail("invalid %s scale length %zu, expected %zu", format_name(d.format), scale_bytes, sexp);
    }
    if (!weight || (sexp && !scales)) fail("weight/scales must not be NULL");
    DeviceGuard dg(device);
    hipStream_t st = (hipStream_t)stream;
    Linear *L = alloc_linear(d, device);
    try {
      DevBuf rw, rs;
      stage_in(rw, weight, weight_bytes, host_io != 0, st);
      if (scale_bytes) stage_in(rs, scales, scale_bytes, host_io != 0, st);
      hip_check(launch_repack(d.format, d.out_dim, d.in_dim, rw.p, rs.p, d.scale_dtype == DIALQ_BF16,
                              (int64_t)scount, (uint8_t *)L->tiles.p, (uint8_t *)L->aux.p,
                              (float *)L->row_scale.p, (float *)L->block_scale.p, st),
                "repack");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
    } catch (...) {
      delete L;
      throw;
    }
    out = L;
  });
  return out;
}

void *dialq_linear_quantize(const dialq_linear_desc *desc, const void *dense, int32_t dense_dtype,
                            int device, int host_io, void *stream, char *error, size_t error_size) {
  Linear *out = nullptr;
  guarded(error, error_size, [&] {
    validate_desc(desc);
    const dialq_linear_desc &d = *desc;
    if (d.format == DIALQ_FORMAT_FP8_ROW || d.format == DIALQ_FORMAT_NVFP4 || d.format == DIALQ_FORMAT_Q6_K)
      fail("%s weights come pre-quantized from the checkpoint; use dialq_linear_create", format_name(d.format));
    if (!dense) fail("dense weight must not be NULL");
    size_t es = dtype_size(dense_dtype);
    size_t wexp, sexp, scount;
    raw_sizes(d, wexp, sexp, scount);
    DeviceGuard dg(device);
    hipStream_t st = (hipStream_t)stream;
    Linear *L = alloc_linear(d, device);
    try {
      DevBuf dd, rw, rs;
      const void *src = dense;
      if (host_io) {
        stage_in(dd, dense, (size_t)(d.out_dim * d.in_dim) * es, true, st);
        src = dd.p;
      }
      rw.alloc(wexp);
      // the quantizer always writes f32 row scales; bf16 storage rounds them
      DevBuf rs32;
      if (d.format == DIALQ_FORMAT_W8A16) rs32.alloc((size_t)d.out_dim * 4);
      else if (sexp) rs.alloc(sexp);
      hip_check(launch_quantize(d.format, src, dense_dtype, d.out_dim, d.in_dim, rw.p,
                                d.format == DIALQ_FORMAT_W8A16 ? rs32.p : rs.p, st),
                "quantize");
      const void *scale_src = d.format == DIALQ_FORMAT_W8A16 ? rs32.p : rs.p;
      if (d.format == DIALQ_FORMAT_W8A16 && d.scale_dtype == DIALQ_BF16) {
        // round the f32 row scales to bf16 storage (RNE); q stays as computed
        // against the f32 scale
        std::vector<float> hs((size_t)d.out_dim);
        hip_check(hipMemcpyAsync(hs.data(), rs32.p, hs.size() * 4, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
        hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
        std::vector<uint16_t> hb(hs.size());
        for (size_t i = 0; i < hs.size(); ++i) {
          uint32_t u;
          memcpy(&u, &hs[i], 4);
          if ((u & 0x7fffffffu) > 0x7f800000u) hb[i] = (uint16_t)((u >> 16) | 0x40u);
          else hb[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        }
        rs.alloc(hb.size() * 2);
        hip_check(hipMemcpyAsync(rs.p, hb.data(), hb.size() * 2, hipMemcpyHostToDevice, st), "hipMemcpyAsync");
        scale_src = rs.p;
        hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
      }
      hip_check(launch_repack(d.format, d.out_dim, d.in_dim, rw.p, scale_src, d.scale_dtype == DIALQ_BF16,
                              (int64_t)scount, (uint8_t *)L->tiles.p, (uint8_t *)L->aux.p,
                              (float *)L->row_scale.p, (float *)L->block_scale.p, st),
                "repack");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
    } catch (...) {
      delete L;
      throw;
    }
    out = L;
  });
  return out;
}

void dialq_linear_destroy(void *linear) {
  Linear *L = (Linear *)linear;
  if (!L) return;
  int prev = -1;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(L->device);
  delete L;
  if (prev >= 0) (void)hipSetDevice(prev);
}

uint64_t dialq_linear_resident_bytes(const void *linear) {
  const Linear *L = (const Linear *)linear;
  if (!L) return 0;
  const dialq_linear_desc &d = L->desc;
  const uint64_t N = (uint64_t)d.out_dim, K = (uint64_t)d.in_dim;
  switch (d.format) {
    case DIALQ_FORMAT_NVFP4: return N * K / 2 + N * K / 16 + 4;
    case DIALQ_FORMAT_FP8_ROW: return N * K + N * 4;
    case DIALQ_FORMAT_W8A16: return N * K + N * (d.scale_dtype == DIALQ_BF16 ? 2 : 4);
    case DIALQ_FORMAT_Q8_0: return N * (K / 32) * 34;
    case DIALQ_FORMAT_Q4_K: return N * (K / 256) * 144;
    case DIALQ_FORMAT_Q6_K: return N * (K / 256) * 210;
    case DIALQ_FORMAT_FP8_BLOCK: return N * K + 4 * ((N + 127) / 128) * ((K + 127) / 128);
    case DIALQ_FORMAT_MXFP4: return N * K / 2 + N * K / 32;
  }
  return 0;
}

uint64_t dialq_linear_device_bytes(const void *linear) {
  const Linear *L = (const Linear *)linear;
  if (!L) return 0;
  return L->tiles.n + L->aux.n + L->row_scale.n + L->block_scale.n + L->act_scratch.n + L->gemv_ws.n +
         L->gemv_cnt.n + L->native_part.n + L->native_cnt.n + L->xstage.n;
}

int dialq_linear_describe(const void *linear, dialq_linear_desc *desc) {
  const Linear *L = (const Linear *)linear;
  if (!L || !desc) return -1;
  *desc = L->desc;
  return 0;
}

int dialq_linear_forward_group(void *const *linears, int32_t n, const void *x, int32_t x_dtype, int64_t rows,
                               void *y, int32_t y_dtype, int32_t path, void *stream, int device_io, char *error,
                               size_t error_size) {
  return guarded(error, error_size, [&] {
    forward_group_impl((Linear *const *)linears, n, x, x_dtype, rows, y, y_dtype, path, stream, device_io);
  });
}

void dialq_debug_set_wait_limit(int64_t polls) { set_gemv_wait_limit(polls); }

int64_t dialq_debug_grouped_launches(void) { return gemv_grouped_launches() + gemm_grouped_launches(); }

int dialq_linear_forward_noalloc(void *linear, const void *x, int32_t x_dtype, int64_t rows, void *y,
                                 int32_t y_dtype, int32_t path, void *stream, char *error, size_t error_size) {
  return guarded(error, error_size, [&] {
    forward_noalloc_impl((Linear *)linear, x, x_dtype, rows, y, y_dtype, path, stream);
  });
}

int dialq_linear_forward(void *linear, const void *x, int32_t x_dtype, int64_t rows, void *y,
                         int32_t y_dtype, void *stream, int device_io, char *error, size_t error_size) {
  return guarded(error, error_size, [&] {
    forward_impl((Linear *)linear, x, x_dtype, rows, y, y_dtype, DIALQ_PATH_AUTO, stream, device_io, false);
  });
}

int dialq_linear_forward_ex(void *linear, const void *x, int32_t x_dtype, int64_t rows, void *y,
                            int32_t y_dtype, int32_t path, void *stream, int device_io, char *error,
                            size_t error_size) {
  return guarded(error, error_size, [&] {
    forward_impl((Linear *)linear, x, x_dtype, rows, y, y_dtype, path, stream, device_io, false);
  });
}

int dialq_linear_forward_swiglu(void *linear, const void *x, int32_t x_dtype, int64_t rows, void *y,
                                int32_t y_dtype, int32_t path, void *stream, int device_io, char *error,
                                size_t error_size) {
  return guarded(error, error_size, [&] {
    forward_impl((Linear *)linear, x, x_dtype, rows, y, y_dtype, path, stream, device_io, false, true);
  });
}

size_t dialq_logits_select_workspace_bytes(int64_t vocab, int64_t n_repeat) {
  if (vocab < 1) return 0;
  const size_t ids = (size_t)(n_repeat > 0 ? n_repeat : 0) * sizeof(uint32_t);
  return (select_workspace_bytes(vocab) + 255) / 256 * 256 + ids;
}

int dialq_logits_select(const void *logits, int32_t dtype, int64_t vocab, const uint32_t *repeat_ids,
                        int64_t n_repeat, float repeat_penalty, float temperature, int32_t rule, int64_t k,
                        uint32_t *out_idx, float *out_val, float *out_stats, void *workspace,
                        size_t workspace_bytes, int32_t device, void *stream, int device_io, char *error,
                        size_t error_size) {
  return guarded(error, error_size, [&] {
    size_t ls = dtype_size(dtype);
    if (rule != DIALQ_SELECT_FIRST_MAX && rule != DIALQ_SELECT_TOTAL_LAST_MAX) fail("unknown selection rule %d", rule);
    if (k < 1 || k > DIALQ_SELECT_MAX_K) fail("k must be in [1, %d], got %lld", DIALQ_SELECT_MAX_K, (long long)k);
    if (vocab < k || vocab > 0xFFFFFFFFLL)
      fail("vocab %lld must be at least k (%lld) and below 2^32", (long long)vocab, (long long)k);
    if (!logits || !out_idx || !out_val || !out_stats) fail("logits and outputs must not be NULL");
    if (n_repeat < 0 || (n_repeat > 0 && !repeat_ids)) fail("repeat context of %lld ids without a pointer", (long long)n_repeat);
    // apply_repeat_penalty_in_place: each distinct id once, ids past the vocabulary ignored
    std::vector<uint32_t> ids;
    if (repeat_penalty != 1.0f && n_repeat > 0) {
      ids.assign(repeat_ids, repeat_ids + n_repeat);
      std::sort(ids.begin(), ids.end());
      ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
      while (!ids.empty() && (int64_t)ids.back() >= vocab) ids.pop_back();
    }
    DeviceGuard dg(device);
    hipStream_t st = (hipStream_t)stream;
    const size_t need = dialq_logits_select_workspace_bytes(vocab, (int64_t)ids.size());
    const size_t ws_off = (select_workspace_bytes(vocab) + 255) / 256 * 256;
    DevBuf own_ws, dl, di, dv, ds;
    void *ws = workspace;
    if (!device_io || !ws) {
      own_ws.alloc(need);
      ws = own_ws.p;
    } else if (workspace_bytes < need) {
      fail("workspace of %zu bytes is smaller than the %zu bytes dialq_logits_select_workspace_bytes asks for",
           workspace_bytes, need);
    }
    const void *lp = logits;
    uint32_t *ip = out_idx;
    float *vp = out_val, *sp = out_stats;
    if (!device_io) {
      stage_in(dl, logits, (size_t)vocab * ls, true, st);
      lp = dl.p;
      di.alloc((size_t)k * 4);
      dv.alloc((size_t)k * 4);
      ds.alloc(8);
      ip = (uint32_t *)di.p;
      vp = (float *)dv.p;
      sp = (float *)ds.p;
    }
    uint32_t *dids = (uint32_t *)((uint8_t *)ws + ws_off);
    if (!ids.empty()) {
      hip_check(hipMemcpyAsync(dids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice, st), "hipMemcpyAsync");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");  // the host list dies with this call
    }
    hip_check(launch_select(lp, dtype, vocab, dids, (int)ids.size(), repeat_penalty, temperature, rule, (int)k, ws,
                            ws_off, ip, vp, sp, st),
              "selection launch");
    if (!device_io) {
      hip_check(hipMemcpyAsync(out_idx, ip, (size_t)k * 4, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
      hip_check(hipMemcpyAsync(out_val, vp, (size_t)k * 4, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
      hip_check(hipMemcpyAsync(out_stats, sp, 8, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
    } else if (!workspace) {
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");  // the call's own workspace is freed on return
    }
  });
}

int dialq_local_q8_forward(void *linear, const void *x, int32_t x_dtype, int64_t rows, void *y,
                           int32_t y_dtype, void *stream, int device_io, char *error,
                           size_t error_size) {
  return guarded(error, error_size, [&] {
    forward_impl((Linear *)linear, x, x_dtype, rows, y, y_dtype, DIALQ_PATH_AUTO, stream, device_io, true);
  });
}

int dialq_linear_dequantize(const void *linear, void *out, int32_t out_dtype, void *stream,
                            int device_io, char *error, size_t error_size) {
  return guarded(error, error_size, [&] {
    const Linear *L = (const Linear *)linear;
    if (!L) fail("linear handle is NULL");
    if (!out) fail("out must not be NULL");
    size_t es = dtype_size(out_dtype);
    DeviceGuard dg(L->device);
    hipStream_t st = (hipStream_t)stream;
    const dialq_linear_desc &d = L->desc;
    size_t bytes = (size_t)(d.out_dim * d.in_dim) * es;
    DevBuf tmp;
    void *dst = out;
    if (!device_io) {
      tmp.alloc(bytes);
      dst = tmp.p;
    }
    FormatGeom fg = format_geom(d.format);
    DequantArgs a;
    a.fmt = d.format;
    a.N = d.out_dim;
    a.K = d.in_dim;
    a.k_chunks = L->k_chunks;
    a.nbk = L->nbk;
    a.chunk = fg.chunk;
    a.tile_bytes = fg.tile_bytes;
    a.tiles = (const uint8_t *)L->tiles.p;
    a.aux = (const uint8_t *)L->aux.p;
    a.row_scale = (const float *)L->row_scale.p;
    a.block_scale = (const float *)L->block_scale.p;
    a.global = L->global;
    a.out = dst;
    a.out_dtype = out_dtype;
    hip_check(launch_dequant(a, st), "dequantize launch");
    if (!device_io) {
      hip_check(hipMemcpyAsync(out, dst, bytes, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
    }
  });
}

int dialq_linear_export(const void *linear, void *weight, size_t weight_bytes, void *scales,
                        size_t scale_bytes, char *error, size_t error_size) {
  return guarded(error, error_size, [&] {
    const Linear *L = (const Linear *)linear;
    if (!L) fail("linear handle is NULL");
    const dialq_linear_desc &d = L->desc;
    size_t wexp, sexp, scount;
    raw_sizes(d, wexp, sexp, scount);
    if (weight_bytes != wexp) fail("export weight buffer has %zu bytes, expected %zu", weight_bytes, wexp);
    if (d.format == DIALQ_FORMAT_W8A16 || d.format == DIALQ_FORMAT_FP8_ROW) {
      // per-row scales are kept as f32; export them in the requested width
      size_t n = (size_t)d.out_dim;
      bool bf16 = d.format == DIALQ_FORMAT_W8A16 && d.scale_dtype == DIALQ_BF16;
      if (scale_bytes != n * (bf16 ? 2 : 4)) fail("export scale buffer has %zu bytes, expected %zu", scale_bytes, n * (bf16 ? 2 : 4));
    } else if (scale_bytes != sexp) {
      fail("export scale buffer has %zu bytes, expected %zu", scale_bytes, sexp);
    }
    DeviceGuard dg(L->device);
    hipStream_t st = nullptr;
    DevBuf rw(wexp), rs(sexp);
    hip_check(launch_unpack(d.format, d.out_dim, d.in_dim, (const uint8_t *)L->tiles.p,
                            (const uint8_t *)L->aux.p, rw.p, rs.p, st),
              "unpack");
    hip_check(hipMemcpyAsync(weight, rw.p, wexp, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    if (d.format == DIALQ_FORMAT_W8A16 || d.format == DIALQ_FORMAT_FP8_ROW) {
      std::vector<float> hs((size_t)d.out_dim);
      hip_check(hipMemcpyAsync(hs.data(), L->row_scale.p, hs.size() * 4, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
      if (d.format == DIALQ_FORMAT_W8A16 && d.scale_dtype == DIALQ_BF16) {
        uint16_t *o = (uint16_t *)scales;
        for (size_t i = 0; i < hs.size(); ++i) {
          uint32_t u;
          memcpy(&u, &hs[i], 4);
          o[i] = (uint16_t)(u >> 16);  // exact: the value came from bf16
        }
      } else {
        memcpy(scales, hs.data(), hs.size() * 4);
      }
    } else if (d.format == DIALQ_FORMAT_FP8_BLOCK) {
      hip_check(hipMemcpyAsync(scales, L->block_scale.p, sexp, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    } else if (sexp) {
      hip_check(hipMemcpyAsync(scales, rs.p, sexp, hipMemcpyDeviceToHost, st), "hipMemcpyAsync");
    }
    hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  });
}

}  // extern "C"

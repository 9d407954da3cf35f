// Prefill GEMM for quantized weights, gfx950.
//
// Reference kernels replaced: dial_w8a16_prefill_f16 (worker_w8a16.rs:186-224),
// dial_nvfp4_prefill_f16 / dial_fp8_prefill_f16 (cuda_quant.rs:135-206) --
// 16x16 scalar-FMA tiles -- and the GGUF prefill route (dequantized F16 copy
// + dense matmul, worker_gguf.rs:425-460, or candle's dequant+matmul).
//
// Weight-only kernel (k_gemm): a 256-thread workgroup computes a
// (16*MS) x (64*NS) output tile.  Activations for one k chunk are staged in
// LDS (bf16 parts; padded rows, conflict-free 16-byte reads) and shared by
// the 4 waves; each wave streams its own NS weight strips straight from the
// resident tiles into registers, unpacks them once per chunk into exact
// bf16 operands and reuses them for all MS row groups.  The next chunk's
// activations and weights are prefetched into registers while the current
// one is multiplied.
//
// Native kernels (k_gemm_fp8 / k_gemm_mxfp4): activations are quantized
// first (per-token E4M3 with an f32 scale; per-32 MXFP4 with E8M0 scales)
// and the product runs on v_mfma_scale_f32_16x16x128_f8f6f4: FP8 with unit
// E8M0 scales and the f32 128x128 weight scale applied per chunk; MXFP4
// with the E8M0 scales of both operands applied by the instruction.
#include "tile_ops.hpp"

namespace dialq {

struct GemmParams {
  WeightView w;
  const void *x;
  void *y;
  int64_t M;
  int y_dtype;
};

template <int FMT, int ACT>
struct GemmShape {
  static constexpr int CHUNK = FmtTraits<FMT>::CHUNK;
  static constexpr int PARTS = ActTraits<ACT>::PARTS;
  static constexpr int STRIDE = CHUNK + 8;  // bf16 elements per LDS row
  static constexpr int ROW_BYTES = STRIDE * 2 * PARTS;
  static constexpr int MS = (16 * 8 * ROW_BYTES <= 65536) ? 8 : ((16 * 4 * ROW_BYTES <= 65536) ? 4 : 2);
  static constexpr int NS = (FMT == DIALQ_FORMAT_Q4_K) ? 2 : 4;
  static constexpr int ROWS = 16 * MS;
  static constexpr int LDS_BYTES = ROWS * ROW_BYTES;
  // 8-element activation pieces per thread per chunk
  static constexpr int PIECES = ROWS * CHUNK / 8 / 256;
};

template <int FMT, int ACT, int MS, int NS>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p) {
  typedef GemmShape<FMT, ACT> S;
  typedef FmtTraits<FMT> T;
  extern __shared__ uint16_t lds[];  // [PARTS][ROWS][STRIDE] bf16
  const WeightView &w = p.w;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t m0 = (int64_t)blockIdx.y * S::ROWS;
  const int64_t s0 = (int64_t)blockIdx.x * (4 * NS) + wave * NS;
  const int64_t kc = w.k_chunks;

  f32x4 acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[i][j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  XOp<ACT> apre[S::PIECES];
  RawTile wpre[NS];
  auto fetch = [&](int64_t c) {
#pragma unroll
    for (int q = 0; q < S::PIECES; ++q) {
      int piece = tid + q * 256;
      int row = piece / (S::CHUNK / 8), kk = (piece % (S::CHUNK / 8)) * 8;
      apre[q] = load_x8<ACT>(p.x, m0 + row, c * S::CHUNK + kk, p.M, w.K);
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int s = (int)(s0 + j < w.n_strips ? s0 + j : w.n_strips - 1);
      const uint8_t *tbase = w.tiles + (size_t)s * kc * (64 * T::LANE) + lane * T::LANE;
      wpre[j] = load_tile_full<FMT>(w, tbase, s, (int)c, lane);
    }
  };

  fetch(0);
  for (int64_t c = 0; c < kc; ++c) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < S::PIECES; ++q) {
      int piece = tid + q * 256;
      int row = piece / (S::CHUNK / 8), kk = (piece % (S::CHUNK / 8)) * 8;
      *(u32x4 *)(lds + row * S::STRIDE + kk) = apre[q].hi;
      if constexpr (S::PARTS == 2) *(u32x4 *)(lds + (S::ROWS + row) * S::STRIDE + kk) = apre[q].lo;
    }
    __syncthreads();
    RawTile cur[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) cur[j] = wpre[j];
    if (c + 1 < kc) fetch(c + 1);

    BOps<FMT> o[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) o[j] = make_bops<FMT>(cur[j]);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      XOp<ACT> xo[T::NX];
#pragma unroll
      for (int t = 0; t < T::NX; ++t) {
        int row = ms * 16 + r, kk = T::xk(t, g);
        xo[t].hi = *(const u32x4 *)(lds + row * S::STRIDE + kk);
        if constexpr (S::PARTS == 2) xo[t].lo = *(const u32x4 *)(lds + (S::ROWS + row) * S::STRIDE + kk);
      }
#pragma unroll
      for (int j = 0; j < NS; ++j) bops_mac<FMT, ACT>(o[j], xo, acc[ms][j]);
    }
  }

#pragma unroll
  for (int j = 0; j < NS; ++j) {
    int64_t n = (s0 + j) * 16 + r;
    if (n >= w.N) continue;
    float scale = epilogue_scale<FMT>(w, n);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int64_t m = m0 + ms * 16 + g * 4 + i;
        if (m < p.M) store_out(p.y, m * w.N + n, p.y_dtype, acc[ms][j][i] * scale);
      }
  }
}

template <int FMT, int ACT>
static hipError_t gemm_dispatch(const WeightView &w, const void *x, int64_t M, void *y, int y_dtype,
                                hipStream_t st) {
  typedef GemmShape<FMT, ACT> S;
  dim3 grid((unsigned)((w.n_strips + 4 * S::NS - 1) / (4 * S::NS)), (unsigned)((M + S::ROWS - 1) / S::ROWS));
  GemmParams p{w, x, y, M, y_dtype};
  k_gemm<FMT, ACT, S::MS, S::NS><<<grid, 256, S::LDS_BYTES, st>>>(p);
  return hipGetLastError();
}

template <int FMT>
static hipError_t gemm_act(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y,
                           int y_dtype, hipStream_t st) {
  switch (x_dtype) {
    case DIALQ_BF16: return gemm_dispatch<FMT, DIALQ_BF16>(w, x, M, y, y_dtype, st);
    case DIALQ_F16: return gemm_dispatch<FMT, DIALQ_F16>(w, x, M, y, y_dtype, st);
    case DIALQ_F32: return gemm_dispatch<FMT, DIALQ_F32>(w, x, M, y, y_dtype, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y,
                       int y_dtype, hipStream_t st) {
  switch (w.fmt) {
    case DIALQ_FORMAT_W8A16: return gemm_act<DIALQ_FORMAT_W8A16>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_FP8_ROW: return gemm_act<DIALQ_FORMAT_FP8_ROW>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_Q8_0: return gemm_act<DIALQ_FORMAT_Q8_0>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_FP8_BLOCK:
      return gemm_act<DIALQ_FORMAT_FP8_BLOCK>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_NVFP4: return gemm_act<DIALQ_FORMAT_NVFP4>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_MXFP4: return gemm_act<DIALQ_FORMAT_MXFP4>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_Q4_K: return gemm_act<DIALQ_FORMAT_Q4_K>(w, x, x_dtype, M, y, y_dtype, st);
  }
  return hipErrorInvalidValue;
}

// ===========================================================================
// Native low-precision prefill.
// ===========================================================================
struct NativeParams {
  WeightView w;
  const uint8_t *xq;  // FP8: [M, k_pad] E4M3; MXFP4: [M, k_pad/2] E2M1 codes
  const void *xs;     // FP8: [M] f32 per-token scale; MXFP4: [M, k_pad/32] E8M0
  int64_t M, k_pad;
  void *y;
  int y_dtype;
};

__device__ __forceinline__ f32x4 mfma_f8f6f4(i32x8 a, i32x8 b, f32x4 c, int sa, int sb, int fmt) {
  if (fmt == 0)
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 4, 0, sa, 0, sb);
}

// FP8_BLOCK: CHUNK 128 = one weight scale block along k.
template <int MS, int NS>
__global__ __launch_bounds__(256) void k_gemm_fp8(NativeParams p) {
  constexpr int ROWS = 16 * MS, STRIDE = 128 + 16;  // bytes per LDS row
  __shared__ uint8_t lds[ROWS * STRIDE];
  const WeightView &w = p.w;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t m0 = (int64_t)blockIdx.y * ROWS;
  const int64_t s0 = (int64_t)blockIdx.x * (4 * NS) + wave * NS;
  const int64_t kc = w.k_chunks;
  constexpr int PIECES = ROWS * 128 / 16 / 256;  // 16-byte pieces per thread

  f32x4 acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[i][j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  u32x4 apre[PIECES];
  RawTile wpre[NS];
  auto fetch = [&](int64_t c) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      int piece = tid + q * 256;
      int row = piece / 8, kb = (piece % 8) * 16;
      int64_t m = m0 + row;
      apre[q] = m < p.M ? *(const u32x4 *)(p.xq + m * p.k_pad + c * 128 + kb) : (u32x4){0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      int64_t s = s0 + j;
      if (s < w.n_strips) wpre[j] = load_tile<DIALQ_FORMAT_FP8_BLOCK>(w.tiles, s * kc + c, lane);
      else wpre[j].a = wpre[j].b = (u32x4){0, 0, 0, 0};
    }
  };

  fetch(0);
  for (int64_t c = 0; c < kc; ++c) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      int piece = tid + q * 256;
      int row = piece / 8, kb = (piece % 8) * 16;
      *(u32x4 *)(lds + row * STRIDE + kb) = apre[q];
    }
    __syncthreads();
    RawTile cur[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) cur[j] = wpre[j];
    if (c + 1 < kc) fetch(c + 1);
    float ws[NS];
    i32x8 bop[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      int64_t s = s0 + j < w.n_strips ? s0 + j : w.n_strips - 1;
      ws[j] = w.block_scale[((s * 16) / 128) * w.nbk + c];
      bop[j] = (i32x8){(int)cur[j].a[0], (int)cur[j].a[1], (int)cur[j].a[2], (int)cur[j].a[3],
                       (int)cur[j].b[0], (int)cur[j].b[1], (int)cur[j].b[2], (int)cur[j].b[3]};
    }
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const uint8_t *ap = lds + (ms * 16 + r) * STRIDE + 32 * g;
      u32x4 a0 = *(const u32x4 *)ap, a1 = *(const u32x4 *)(ap + 16);
      i32x8 aop = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                   (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        f32x4 t = mfma_f8f6f4(aop, bop[j], (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 127, 127, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ms][j][i] = __builtin_fmaf(ws[j], t[i], acc[ms][j][i]);
      }
    }
  }

  const float *xs = (const float *)p.xs;
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int64_t m = m0 + ms * 16 + g * 4 + i;
      if (m >= p.M) continue;
      float sx = xs[m];
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        int64_t n = (s0 + j) * 16 + r;
        if (n < w.N) store_out(p.y, m * w.N + n, p.y_dtype, acc[ms][j][i] * sx);
      }
    }
}

// MXFP4: CHUNK 128 = four 32-blocks; lane group g holds block g.
template <int MS, int NS>
__global__ __launch_bounds__(256) void k_gemm_mxfp4(NativeParams p) {
  constexpr int ROWS = 16 * MS, STRIDE = 64 + 16;  // code bytes per LDS row
  __shared__ uint8_t lds[ROWS * STRIDE];
  __shared__ uint32_t lds_s[ROWS];  // 4 E8M0 scales per row
  const WeightView &w = p.w;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t m0 = (int64_t)blockIdx.y * ROWS;
  const int64_t s0 = (int64_t)blockIdx.x * (4 * NS) + wave * NS;
  const int64_t kc = w.k_chunks;
  constexpr int PIECES = (ROWS * 64 / 16 + 255) / 256;
  const uint8_t *xsc = (const uint8_t *)p.xs;

  f32x4 acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[i][j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  u32x4 apre[PIECES];
  uint32_t spre = 0;
  RawTile wpre[NS];
  auto fetch = [&](int64_t c) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      int piece = tid + q * 256;
      int row = piece / 4, kb = (piece % 4) * 16;
      int64_t m = m0 + row;
      apre[q] = (row < ROWS && m < p.M) ? *(const u32x4 *)(p.xq + m * (p.k_pad / 2) + c * 64 + kb)
                                        : (u32x4){0, 0, 0, 0};
    }
    if (tid < ROWS) {
      int64_t m = m0 + tid;
      spre = m < p.M ? *(const uint32_t *)(xsc + m * (p.k_pad / 32) + c * 4) : 0u;
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      int64_t s = s0 + j;
      if (s < w.n_strips) wpre[j] = load_tile<DIALQ_FORMAT_MXFP4>(w.tiles, s * kc + c, lane);
      else wpre[j].a = wpre[j].b = (u32x4){0, 0, 0, 0};
    }
  };

  fetch(0);
  for (int64_t c = 0; c < kc; ++c) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      int piece = tid + q * 256;
      int row = piece / 4, kb = (piece % 4) * 16;
      if (row < ROWS) *(u32x4 *)(lds + row * STRIDE + kb) = apre[q];
    }
    if (tid < ROWS) lds_s[tid] = spre;
    __syncthreads();
    RawTile cur[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) cur[j] = wpre[j];
    if (c + 1 < kc) fetch(c + 1);
    i32x8 bop[NS];
    int bsc[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      int64_t s = s0 + j < w.n_strips ? s0 + j : w.n_strips - 1;
      bsc[j] = w.aux[(s * kc + c) * 64 + r * 4 + g];
      bop[j] = (i32x8){(int)cur[j].a[0], (int)cur[j].a[1], (int)cur[j].a[2], (int)cur[j].a[3], 0, 0, 0, 0};
    }
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      int row = ms * 16 + r;
      u32x4 a0 = *(const u32x4 *)(lds + row * STRIDE + 16 * g);
      i32x8 aop = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], 0, 0, 0, 0};
      int asc = (lds_s[row] >> (8 * g)) & 0xff;
#pragma unroll
      for (int j = 0; j < NS; ++j) acc[ms][j] = mfma_f8f6f4(aop, bop[j], acc[ms][j], asc, bsc[j], 4);
    }
  }

#pragma unroll
  for (int j = 0; j < NS; ++j) {
    int64_t n = (s0 + j) * 16 + r;
    if (n >= w.N) continue;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int64_t m = m0 + ms * 16 + g * 4 + i;
        if (m < p.M) store_out(p.y, m * w.N + n, p.y_dtype, acc[ms][j][i]);
      }
  }
}

hipError_t launch_gemm_native(const WeightView &w, const uint8_t *xq, const void *xs, int64_t M,
                              int64_t k_pad, void *y, int y_dtype, hipStream_t st) {
  constexpr int MS = 8, NS = 4;
  dim3 grid((unsigned)((w.n_strips + 4 * NS - 1) / (4 * NS)), (unsigned)((M + 16 * MS - 1) / (16 * MS)));
  NativeParams p{w, xq, xs, M, k_pad, y, y_dtype};
  if (w.fmt == DIALQ_FORMAT_FP8_BLOCK) {
    k_gemm_fp8<MS, NS><<<grid, 256, 0, st>>>(p);
  } else if (w.fmt == DIALQ_FORMAT_MXFP4) {
    k_gemm_mxfp4<MS, NS><<<grid, 256, 0, st>>>(p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace dialq

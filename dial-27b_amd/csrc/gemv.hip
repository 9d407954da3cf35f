// Decode GEMV for quantized weights, gfx950: rows M = 1..16 per 16-row
// group, up to 4 groups (64 rows) per launch.
//
// Reference kernels replaced: dial_w8a16_decode_f16 (worker_w8a16.rs:146-184),
// dial_nvfp4_decode_f16 / dial_fp8_decode_f16 (cuda_quant.rs:67-133) and
// candle's MMVQ for GGUF rows <= 8 (reached from worker_gguf.rs:584-605).
// Those read one weight byte per thread per step and reduce with shuffles.
// Here each wavefront streams resident 1-2 KB tiles with one coalesced
// 16/32-byte load per lane, unpacks them in registers into exact bf16 MFMA
// operands (tile_ops.hpp) and lets v_mfma_f32_16x16x32_bf16 accumulate; the
// weight bytes are read exactly once per launch.
//
// A workgroup owns one 16-row strip.  Its W waves take interleaved k chunks
// (wave w: chunks w, w+W, ...; U chunks in flight per wave) and reduce
// through LDS at the end in a fixed order, so results are deterministic.
#include "tile_ops.hpp"

namespace dialq {

struct GemvParams {
  WeightView w;
  const void *x;
  void *y;
  int64_t M;       // total rows of x / y
  int64_t m_base;  // first row handled by this launch
  int y_dtype;
};

template <int FMT, int ACT, int MG, int U>
__global__ __launch_bounds__(1024) void k_gemv(GemvParams p) {
  extern __shared__ float red[];
  typedef FmtTraits<FMT> T;
  const WeightView &w = p.w;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int W = blockDim.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t s = blockIdx.x;
  const int64_t kc = w.k_chunks;

  f32x4 acc[MG];
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) acc[mg] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  for (int64_t c0 = wave; c0 < kc; c0 += (int64_t)W * U) {
    RawTile tl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t c = c0 + (int64_t)u * W;
      if (c < kc) tl[u] = load_tile<FMT>(w.tiles, s * kc + c, lane);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t c = c0 + (int64_t)u * W;
      if (c < kc) {
        XOp<ACT> xo[MG][T::NX];
#pragma unroll
        for (int mg = 0; mg < MG; ++mg)
#pragma unroll
          for (int t = 0; t < T::NX; ++t)
            xo[mg][t] = load_x8<ACT>(p.x, p.m_base + mg * 16 + r, c * T::CHUNK + T::xk(t, g), p.M, w.K);
        BOps<FMT> o = make_bops<FMT>(tl[u], w, s, c, lane);
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) bops_mac<FMT, ACT>(o, xo[mg], acc[mg]);
      }
    }
  }

  // cross-wave reduction in a fixed order
  float *mine = red + (size_t)wave * 64 * 4 * MG;
#pragma unroll
  for (int mg = 0; mg < MG; ++mg)
#pragma unroll
    for (int i = 0; i < 4; ++i) mine[(mg * 4 + i) * 64 + lane] = acc[mg][i];
  __syncthreads();
  if (wave == 0) {
    const int64_t n = s * 16 + r;
    const float scale = epilogue_scale<FMT>(w, n);
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = 0.0f;
        for (int ww = 0; ww < W; ++ww) v += red[(size_t)ww * 64 * 4 * MG + (mg * 4 + i) * 64 + lane];
        int64_t m = p.m_base + mg * 16 + g * 4 + i;
        if (m < p.M && n < w.N) store_out(p.y, m * w.N + n, p.y_dtype, v * scale);
      }
  }
}

template <int FMT, int ACT>
static hipError_t gemv_dispatch(const WeightView &w, const void *x, int64_t M, void *y, int y_dtype,
                                hipStream_t st) {
  // Waves per workgroup: enough strips x waves to cover the 256 CUs several
  // times over, without giving a wave fewer than ~8 chunks.
  int waves = 4;
  while (waves < 16 && w.n_strips * waves < 4096 && w.k_chunks >= (int64_t)waves * 16) waves *= 2;
  dim3 grid((unsigned)w.n_strips), block((unsigned)(64 * waves));
  for (int64_t mb = 0; mb < M; mb += 64) {
    GemvParams p{w, x, y, M, mb, y_dtype};
    int64_t rem = M - mb;
    if (rem <= 16) {
      size_t lds = (size_t)waves * 64 * 4 * 1 * sizeof(float);
      k_gemv<FMT, ACT, 1, 4><<<grid, block, lds, st>>>(p);
    } else if (rem <= 32) {
      size_t lds = (size_t)waves * 64 * 4 * 2 * sizeof(float);
      k_gemv<FMT, ACT, 2, 2><<<grid, block, lds, st>>>(p);
    } else {
      size_t lds = (size_t)waves * 64 * 4 * 4 * sizeof(float);
      k_gemv<FMT, ACT, 4, 1><<<grid, block, lds, st>>>(p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int FMT>
static hipError_t gemv_act(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y,
                           int y_dtype, hipStream_t st) {
  switch (x_dtype) {
    case DIALQ_BF16: return gemv_dispatch<FMT, DIALQ_BF16>(w, x, M, y, y_dtype, st);
    case DIALQ_F16: return gemv_dispatch<FMT, DIALQ_F16>(w, x, M, y, y_dtype, st);
    case DIALQ_F32: return gemv_dispatch<FMT, DIALQ_F32>(w, x, M, y, y_dtype, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y,
                       int y_dtype, hipStream_t st) {
  switch (w.fmt) {
    case DIALQ_FORMAT_W8A16: return gemv_act<DIALQ_FORMAT_W8A16>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_FP8_ROW: return gemv_act<DIALQ_FORMAT_FP8_ROW>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_Q8_0: return gemv_act<DIALQ_FORMAT_Q8_0>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_FP8_BLOCK:
      return gemv_act<DIALQ_FORMAT_FP8_BLOCK>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_NVFP4: return gemv_act<DIALQ_FORMAT_NVFP4>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_MXFP4: return gemv_act<DIALQ_FORMAT_MXFP4>(w, x, x_dtype, M, y, y_dtype, st);
    case DIALQ_FORMAT_Q4_K: return gemv_act<DIALQ_FORMAT_Q4_K>(w, x, x_dtype, M, y, y_dtype, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace dialq

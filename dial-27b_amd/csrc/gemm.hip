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
  // chunks per pipeline stage (one for the formats whose per-block scales
  // need extra registers)
  static constexpr int KS = (CHUNK == 64 && FMT != DIALQ_FORMAT_Q8_0) ? 2 : 1;
  static constexpr int SK = KS * CHUNK;                // k per stage
  static constexpr int STRIDE = SK + 8;                // bf16 elements per LDS row
  static constexpr int MS = (FMT == DIALQ_FORMAT_Q4_K) ? 4 : 8;  // 16-row groups per workgroup
  static constexpr int NS = (FMT == DIALQ_FORMAT_Q4_K) ? 2 : 4;  // 16-col strips per wave
  static constexpr int ROWS = 16 * MS;
  static constexpr int BUF = PARTS * ROWS * STRIDE;   // bf16 elements per LDS buffer
  static constexpr int LDS_BYTES = 2 * BUF * 2;
  static constexpr int PIECES = ROWS * SK / 8 / 256;  // 8-element activation pieces per thread
};

// Weight tile (strip s, chunk c) with its scales; default cache policy (the
// workgroups of the other row blocks read the same tiles).
template <int FMT>
__device__ __forceinline__ RawTile gemm_tile(const WeightView &w, rsrc_t rt, rsrc_t ra, int s, int c, bool valid,
                                             int lane) {
  typedef FmtTraits<FMT> T;
  const int r = lane & 15, g = lane >> 4;
  const uint32_t tidx = (uint32_t)s * (uint32_t)w.k_chunks + (uint32_t)c;
  const uint32_t off = valid ? tidx * (64 * T::LANE) + lane * T::LANE : kOOB;
  RawTile t;
  t.a = bload16(rt, off);
  t.b = (u32x4){0, 0, 0, 0};
  if constexpr (T::LANE == 32) t.b = bload16(rt, valid ? off + 16 : kOOB);
  t.s0 = 0;
  t.hdr = (u32x4){0, 0, 0, 0};
  if constexpr (FMT == DIALQ_FORMAT_Q8_0) t.s0 = bload4(ra, valid ? tidx * 64 + r * 4 : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_Q4_K) t.hdr = bload16(ra, valid ? tidx * 256 + r * 16 : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_NVFP4) t.s0 = bload2(ra, valid ? tidx * 128 + r * 8 + 2 * g : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_MXFP4) t.s0 = bload1(ra, valid ? tidx * 64 + r * 4 + g : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_FP8_BLOCK)
    t.s0 = bload4(ra, valid ? ((uint32_t)((s * 16) / 128) * (uint32_t)w.nbk + (uint32_t)c) * 4 : kOOB);
  return t;
}

// XCD-aware tile order.  Workgroups are dispatched round-robin over the 8
// XCDs (each with its own L2), so hardware id b runs on XCD b % 8.  The map
// gives every XCD a contiguous run of logical tiles, and logical tiles go in
// panels of kPanel row blocks, column-major inside the panel: the ~32
// workgroups an XCD runs at once cover about 4 row blocks x 8 column tiles
// and share their activation and weight tiles in that XCD's L2.
constexpr int kXcds = 8, kPanel = 4;
#ifndef GEMM32_MT
#define GEMM32_MT 2  // 32-row MFMA tiles per workgroup in the 32x32 kernel
#endif
#ifndef GEMM32_KS
#define GEMM32_KS 1  // 64-k chunks per pipeline stage in the 32x32 kernel
#endif
#ifndef GEMM32_OCC
#define GEMM32_OCC 3  // workgroups per CU the 32x32 kernel is built for
#endif
__device__ __forceinline__ void tile_of(int b, int G, int nt, int mt, int &tm, int &tn) {
  const int q = G / kXcds, rem = G % kXcds, xcd = b % kXcds, local = b / kXcds;
  const int L = xcd * q + (xcd < rem ? xcd : rem) + local;  // bijection onto [0, G)
  const int panel = L / (kPanel * nt), i = L - panel * (kPanel * nt);
  const int pm = (mt - panel * kPanel) < kPanel ? (mt - panel * kPanel) : kPanel;  // rows in this panel
  tm = panel * kPanel + i % pm;
  tn = i / pm;
}

// Weight-only prefill GEMM.  A 256-thread workgroup computes a
// (16*MS) x (64*NS) tile of y; wave v owns strips s0 + v*NS .. + NS-1.
// The k loop runs in stages of KS chunks, software-pipelined:
//   * activations of stage t+1 sit in registers (raw input dtype) while
//     stage t is multiplied; after the stage's single barrier they are
//     converted into bf16 operand parts and written to the other LDS buffer,
//     and the loads of stage t+2 are issued into the same registers;
//   * weight tiles live in a two-stage register ring: the slot of stage t is
//     refilled with stage t+2 right after each tile has been multiplied.
// All global reads are buffer loads; out-of-range rows, k and strips read
// zeros, so no load is conditional.
template <int FMT, int ACT, int MS, int NS>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p) {
  typedef GemmShape<FMT, ACT> S;
  typedef FmtTraits<FMT> T;
  constexpr int KS = S::KS, BY = ActTraits<ACT>::BYTES;
  extern __shared__ uint16_t lds[];  // [2][PARTS][ROWS][STRIDE] bf16
  const WeightView &w = p.w;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r = lane & 15;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, (int)((w.n_strips + 4 * NS - 1) / (4 * NS)), (int)((p.M + S::ROWS - 1) / S::ROWS), tm,
          tn);
  const int m0 = tm * S::ROWS;
  const int s0 = tn * (4 * NS) + wave * NS;
  const int kc = (int)w.k_chunks;
  const int K = (int)w.K;
  const int nstage = (kc + KS - 1) / KS;
  const int64_t total = w.n_strips * w.k_chunks;

  const rsrc_t rt = make_rsrc(w.tiles, (uint32_t)(total * 64 * T::LANE));
  rsrc_t ra = rt;
  if constexpr (FMT == DIALQ_FORMAT_Q8_0 || FMT == DIALQ_FORMAT_MXFP4)
    ra = make_rsrc(w.aux, (uint32_t)(total * 64));
  else if constexpr (FMT == DIALQ_FORMAT_Q4_K)
    ra = make_rsrc(w.aux, (uint32_t)(total * 256));
  else if constexpr (FMT == DIALQ_FORMAT_NVFP4)
    ra = make_rsrc(w.aux, (uint32_t)(total * 128));
  else if constexpr (FMT == DIALQ_FORMAT_FP8_BLOCK)
    ra = make_rsrc(w.block_scale, (uint32_t)(((w.N + 127) / 128) * w.nbk * 4));
  const int mrows = (int)((p.M - m0) < S::ROWS ? (p.M - m0) : S::ROWS);
  const rsrc_t rx = make_rsrc((const uint8_t *)p.x + (int64_t)m0 * K * BY, (uint32_t)((int64_t)mrows * K * BY));

  // activation piece q of a stage: row, k offset within the stage
  auto apiece = [&](int q, int &row, int &kk) {
    const int piece = tid + q * 256;
    row = piece / (S::SK / 8);
    kk = (piece % (S::SK / 8)) * 8;
  };
  XRaw<ACT> apre[S::PIECES];
  auto fetch_a = [&](int st) {
#pragma unroll
    for (int q = 0; q < S::PIECES; ++q) {
      int row, kk;
      apiece(q, row, kk);
      const int k = st * S::SK + kk;
      apre[q] = xraw_load<ACT>(rx, (st < nstage && k < K) ? (uint32_t)((row * K + k) * BY) : kOOB);
    }
  };
  auto store_a = [&](int buf) {
    uint16_t *base = lds + buf * S::BUF;
#pragma unroll
    for (int q = 0; q < S::PIECES; ++q) {
      int row, kk;
      apiece(q, row, kk);
      const XOp<ACT> o = xraw_to_op<ACT>(apre[q]);
      *(u32x4 *)(base + row * S::STRIDE + kk) = o.hi;
      if constexpr (S::PARTS == 2) *(u32x4 *)(base + (S::ROWS + row) * S::STRIDE + kk) = o.lo;
    }
  };
  RawTile wb[2][KS][NS];
  auto fetch_b = [&](RawTile (&slot)[KS][NS], int st) {
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        const int c = st * KS + j, sn = s0 + n;
        const bool valid = st < nstage && c < kc && sn < w.n_strips;
        slot[j][n] = gemm_tile<FMT>(w, rt, ra, valid ? sn : 0, valid ? c : 0, valid, lane);
      }
  };

  f32x4 acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int n = 0; n < NS; ++n) acc[i][n] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  // prologue: stage 0 into LDS buffer 0, stage 1 in registers, weights of
  // stages 0 and 1 in the ring
  fetch_b(wb[0], 0);
  fetch_b(wb[1], 1);
  fetch_a(0);
  store_a(0);
  fetch_a(1);

  auto stage = [&](RawTile (&slot)[KS][NS], int st) {
    __syncthreads();  // buffer st&1 written; buffer (st+1)&1 no longer read
    store_a((st + 1) & 1);
    fetch_a(st + 2);
    const uint16_t *base = lds + (st & 1) * S::BUF;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      BOps<FMT> o[NS];
#pragma unroll
      for (int n = 0; n < NS; ++n) o[n] = make_bops<FMT>(slot[j][n]);
      // refill this chunk's ring slot with stage st+2 as soon as it is unpacked
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        const int c = (st + 2) * KS + j, sn = s0 + n;
        const bool valid = st + 2 < nstage && c < kc && sn < w.n_strips;
        slot[j][n] = gemm_tile<FMT>(w, rt, ra, valid ? sn : 0, valid ? c : 0, valid, lane);
      }
      if constexpr (FMT == DIALQ_FORMAT_W8A16 || FMT == DIALQ_FORMAT_FP8_ROW || FMT == DIALQ_FORMAT_NVFP4 ||
                    FMT == DIALQ_FORMAT_MXFP4) {
        // k step outermost: the two updates of one accumulator are MS*NS
        // MFMAs apart, so the matrix pipe never waits on its own result
#pragma unroll
        for (int t = 0; t < T::NX; ++t)
#pragma unroll
          for (int part = 0; part < S::PARTS; ++part)
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
              const int row = ms * 16 + r, kk = j * S::CHUNK + T::xk(t, g);
              const u32x4 xa = *(const u32x4 *)(base + (part * S::ROWS + row) * S::STRIDE + kk);
#pragma unroll
              for (int n = 0; n < NS; ++n) acc[ms][n] = mfma_bf16(xa, o[n].b[t], acc[ms][n]);
            }
      } else {
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
          XOp<ACT> xo[T::NX];
#pragma unroll
          for (int t = 0; t < T::NX; ++t) {
            const int row = ms * 16 + r, kk = j * S::CHUNK + T::xk(t, g);
            xo[t].hi = *(const u32x4 *)(base + row * S::STRIDE + kk);
            if constexpr (S::PARTS == 2) xo[t].lo = *(const u32x4 *)(base + (S::ROWS + row) * S::STRIDE + kk);
          }
#pragma unroll
          for (int n = 0; n < NS; ++n) bops_mac<FMT, ACT>(o[n], xo, acc[ms][n]);
        }
      }
    }
  };
  int st = 0;
  for (; st + 1 < nstage; st += 2) {
    stage(wb[0], st);
    stage(wb[1], st + 1);
  }
  if (st < nstage) stage(wb[0], st);

#pragma unroll
  for (int n = 0; n < NS; ++n) {
    const int64_t col = (int64_t)(s0 + n) * 16 + r;
    if (col >= w.N) continue;
    const float scale = epilogue_scale<FMT>(w, col);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ms * 16 + g * 4 + i;
        if (m < p.M) store_out(p.y, m * w.N + col, p.y_dtype, acc[ms][n][i] * scale);
      }
  }
}

// ---------------------------------------------------------------------------
// Byte formats (W8A16, FP8_ROW) on v_mfma_f32_32x32x16_bf16, whose issue rate
// on gfx950 is twice that of the 16x16x32 form per flop (measured: 2.26 vs
// 1.25 PFLOP/s of independent MFMAs).  A 256-thread workgroup computes a
// (32*MT) x 256 tile of y; wave v owns columns 64v .. 64v+63 as two
// 32-column MFMA tiles (strips s0+2q, s0+2q+1) and all rows as MT 32-row
// MFMA tiles.  MT = 2 with one 64-k chunk per stage keeps a wave under 171
// registers, so three workgroups share a CU and hide each other's waits.  The B operand of a 16-k step is the
// 8 weight bytes of row n = lane % 32, k = 8*(lane / 32) .. +7, which sit
// contiguously in the resident 16-row tile (lane-slot (k/16)*16 + r, byte
// k % 16), so each lane reads them with one 8-byte buffer load and converts
// them exactly to bf16.  A operands come from the same double-buffered LDS
// stage as the 16x16 kernel; weights ride a two-stage register ring.
// C layout of the 32x32 tile: lane l, value v -> row 8(v/4) + 4(l/32) + v%4,
// column l % 32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

template <int FMT, int ACT, int MT, int KS, int OCC>
__global__ __launch_bounds__(256, OCC) void k_gemm32(GemmParams p) {
  constexpr int CHUNK = 64, SK = KS * CHUNK, STEPS = SK / 16;
  constexpr int PARTS = ActTraits<ACT>::PARTS, BY = ActTraits<ACT>::BYTES;
  constexpr int ROWS = 32 * MT, STRIDE = SK + 8, BUF = PARTS * ROWS * STRIDE;
  constexpr int NQ = 2, PIECES = ROWS * SK / 8 / 256;
  extern __shared__ uint16_t lds[];  // [2][PARTS][ROWS][STRIDE] bf16
  const WeightView &w = p.w;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, r = lane & 15, sub = (lane >> 4) & 1;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, (int)((w.n_strips + 15) / 16), (int)((p.M + ROWS - 1) / ROWS), tm, tn);
  const int m0 = tm * ROWS;
  const int s0 = tn * 16 + wave * 4;
  const int kc = (int)w.k_chunks, K = (int)w.K;
  const int nstage = (kc + KS - 1) / KS;
  const int64_t total = w.n_strips * w.k_chunks;
  const rsrc_t rt = make_rsrc(w.tiles, (uint32_t)(total * 1024));
  const int mrows = (int)((p.M - m0) < ROWS ? (p.M - m0) : ROWS);
  const rsrc_t rx = make_rsrc((const uint8_t *)p.x + (int64_t)m0 * K * BY, (uint32_t)((int64_t)mrows * K * BY));

  XRaw<ACT> apre[PIECES];
  auto fetch_a = [&](int st) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int piece = tid + q * 256, row = piece / (SK / 8), kk = (piece % (SK / 8)) * 8;
      const int k = st * SK + kk;
      apre[q] = xraw_load<ACT>(rx, (st < nstage && k < K) ? (uint32_t)((row * K + k) * BY) : kOOB);
    }
  };
  auto store_a = [&](int buf) {
    uint16_t *base = lds + buf * BUF;
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int piece = tid + q * 256, row = piece / (SK / 8), kk = (piece % (SK / 8)) * 8;
      const XOp<ACT> o = xraw_to_op<ACT>(apre[q]);
      *(u32x4 *)(base + row * STRIDE + kk) = o.hi;
      if constexpr (PARTS == 2) *(u32x4 *)(base + (ROWS + row) * STRIDE + kk) = o.lo;
    }
  };
  // weight bytes of (stage st, 16-k step j, column tile q) for this lane
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  auto bload = [&](int st, int j, int q) -> u32x2 {
    const int c = st * KS + j / 4, strip = s0 + 2 * q + sub;
    const bool valid = st < nstage && c < kc && strip < w.n_strips;
    const uint32_t off = valid ? ((uint32_t)strip * (uint32_t)kc + (uint32_t)c) * 1024u +
                                     (uint32_t)(((j % 4) * 16 + r) * 16 + 8 * h)
                               : kOOB;
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rt, (int)off, 0, 0));
  };
  u32x2 wb[2][STEPS][NQ];
  auto fetch_b = [&](u32x2 (&slot)[STEPS][NQ], int st) {
#pragma unroll
    for (int j = 0; j < STEPS; ++j)
#pragma unroll
      for (int q = 0; q < NQ; ++q) slot[j][q] = bload(st, j, q);
  };

  f32x16 acc[MT][NQ];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][q][v] = 0.0f;

  fetch_b(wb[0], 0);
  fetch_b(wb[1], 1);
  fetch_a(0);
  store_a(0);
  fetch_a(1);

  auto stage = [&](u32x2 (&slot)[STEPS][NQ], int st) {
    __syncthreads();  // buffer st&1 written; buffer (st+1)&1 no longer read
    store_a((st + 1) & 1);
    fetch_a(st + 2);
    const uint16_t *base = lds + (st & 1) * BUF;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
      u32x4 b[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        if constexpr (FMT == DIALQ_FORMAT_W8A16) b[q] = i8x8_to_bf16(slot[j][q][0], slot[j][q][1]);
        else b[q] = e4m3x8_to_bf16(slot[j][q][0], slot[j][q][1]);
        slot[j][q] = bload(st + 2, j, q);  // refill with stage st+2
      }
#pragma unroll
      for (int part = 0; part < PARTS; ++part)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = mt * 32 + (lane & 31), kk = j * 16 + 8 * h;
          const u32x4 a = *(const u32x4 *)(base + (part * ROWS + row) * STRIDE + kk);
#pragma unroll
          for (int q = 0; q < NQ; ++q) acc[mt][q] = mfma32(a, b[q], acc[mt][q]);
        }
    }
  };
  int st = 0;
  for (; st + 1 < nstage; st += 2) {
    stage(wb[0], st);
    stage(wb[1], st + 1);
  }
  if (st < nstage) stage(wb[0], st);

#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int64_t col = (int64_t)(s0 + 2 * q) * 16 + (lane & 31);
    if (col >= w.N) continue;
    const float scale = w.row_scale[col];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + mt * 32 + 8 * (v / 4) + 4 * h + (v % 4);
        if (m < p.M) store_out(p.y, m * w.N + col, p.y_dtype, acc[mt][q][v] * scale);
      }
  }
}

template <int FMT, int ACT>
static hipError_t gemm_dispatch(const WeightView &w, const void *x, int64_t M, void *y, int y_dtype,
                                hipStream_t st) {
  typedef GemmShape<FMT, ACT> S;
  if ((int64_t)S::ROWS * w.K * ActTraits<ACT>::BYTES > 0xffffffffLL) return hipErrorInvalidValue;
  if constexpr (FMT == DIALQ_FORMAT_W8A16 || FMT == DIALQ_FORMAT_FP8_ROW) {
    if (w.n_strips * w.k_chunks * 1024 <= 0xffffffffLL) {
      constexpr int MT = GEMM32_MT, KS = GEMM32_KS, ROWS = 32 * MT;
      constexpr int BUF = ActTraits<ACT>::PARTS * ROWS * (KS * 64 + 8);
      dim3 grid((unsigned)(((w.n_strips + 15) / 16) * ((M + ROWS - 1) / ROWS)));
      GemmParams p{w, x, y, M, y_dtype};
      k_gemm32<FMT, ACT, MT, KS, GEMM32_OCC><<<grid, 256, 2 * BUF * 2, st>>>(p);
      return hipGetLastError();
    }
  }
  dim3 grid((unsigned)(((w.n_strips + 4 * S::NS - 1) / (4 * S::NS)) * ((M + S::ROWS - 1) / S::ROWS)));
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

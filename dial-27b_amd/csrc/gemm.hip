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
// Native kernel (k_gemm_native, FP8_BLOCK and MXFP4): activations are
// quantized first (per-token E4M3 with an f32 scale; per-32 MXFP4 with E8M0
// scales) and the product runs on v_mfma_scale_f32_32x32x64_f8f6f4, with the
// E8M0 scales of both operands applied by the instruction.
#include <atomic>

#include "tile_ops.hpp"

namespace dialq {

std::atomic<int64_t> g_prefill_grouped_launches{0};  // grouped prefill launches made (a test hook)

// Grouped launch (nm > 1): weights that share x and K, their column tiles
// laid end to end -- member j owns global column tiles [tbase[j],
// tbase[j + 1]) and writes through ym[j] with its view's output stride.
struct GemmGroup {
  int nm = 0;
  int tbase[kGemmMaxGroup + 1] = {};
  WeightView wm[kGemmMaxGroup] = {};
  void *ym[kGemmMaxGroup] = {};
};

// The member owning global column tile tn.
__device__ __forceinline__ int group_member(const GemmGroup &g, int tn) {
  int j = 0;
  while (j + 1 < g.nm && tn >= g.tbase[j + 1]) ++j;
  return j;
}

struct GemmParams {
  WeightView w;
  const void *x;
  void *y;
  int64_t M;
  int y_dtype;
  // Split-K (k_gemm32, k_gemm_kq; P > 1): each tile's chunks split into P
  // pieces, one workgroup each; partial tiles in `part` ([tiles][P][rows x
  // 256]), one arrival counter per tile in `cnt` (zero between launches).
  int P = 1;
  float *part = nullptr;
  int *cnt = nullptr;
  // Tail split (W > 0, P > 1): tiles [0, W) whole, the rest in P pieces;
  // `part` / `cnt` are then indexed by the split tile's index past W.
  int W = 0;
  GemmGroup g;  // k_gemm32, k_gemm_kq
  // k_gemm_kq: per-row output multipliers (bf16 activations scaled into f16
  // range, 2^e per row); null = 1
  const float *yrow = nullptr;
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
  static constexpr bool KQ = FMT == DIALQ_FORMAT_Q4_K || FMT == DIALQ_FORMAT_Q6_K;
  static constexpr int MS = KQ ? 2 : 8;  // 16-row groups per workgroup
  // 16-col strips per wave.  Q6_K: one -- its three-plane tiles, 8 operands
  // and 16 scales per strip spill at two strips (f16 / f32 activations:
  // ~4 KB of scratch per lane)
  static constexpr int NS = FMT == DIALQ_FORMAT_Q6_K ? 1 : (KQ ? 2 : 4);
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
  RawTile t;
  t.s0 = 0;
  t.hdr = (u32x4){0, 0, 0, 0};
  if constexpr (FMT == DIALQ_FORMAT_Q6_K) {  // three 1 KB planes, 16 B per lane each
    const uint32_t off = valid ? tidx * 3072 + lane * 16 : kOOB;
    t.a = bload16(rt, off);
    t.b = bload16(rt, valid ? off + 1024 : kOOB);
    t.hdr = bload16(rt, valid ? off + 2048 : kOOB);
    t.sc = bload16(ra, valid ? tidx * 288 + r * 16 : kOOB);
    t.s0 = bload2(ra, valid ? tidx * 288 + 256 + r * 2 : kOOB);
    return t;
  }
  const uint32_t off = valid ? tidx * (64 * T::LANE) + lane * 16 : kOOB;  // plane 0
  t.a = bload16(rt, off);
  t.b = (u32x4){0, 0, 0, 0};
  if constexpr (T::LANE == 32) t.b = bload16(rt, valid ? off + 1024 : kOOB);  // plane 1
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
#ifndef GEMMKQ_MT
#define GEMMKQ_MT 4  // 32-row MFMA tiles per workgroup in the GGUF (Q4_K, Q8_0) prefill kernel
#endif
#ifndef GEMMKQ_OCC
#define GEMMKQ_OCC 2  // workgroups per CU the GGUF prefill kernel is built for
#endif
#ifndef GEMM32_OCC
#define GEMM32_OCC 3  // workgroups per CU the 32x32 kernel is built for
#endif
// Rank of workgroup b among G such that each XCD (b % kXcds) holds a
// contiguous run of ranks: a bijection onto [0, G).
__device__ __forceinline__ int xcd_rank(int b, int G) {
  const int q = G / kXcds, rem = G % kXcds, xcd = b % kXcds, local = b / kXcds;
  return xcd * q + (xcd < rem ? xcd : rem) + local;
}
// Logical tile L -> (row block, column tile): panels of kPanel row blocks,
// column-major inside a panel.
__device__ __forceinline__ void tile_coords(int L, int nt, int mt, int &tm, int &tn) {
  const int panel = L / (kPanel * nt), i = L - panel * (kPanel * nt);
  const int pm = (mt - panel * kPanel) < kPanel ? (mt - panel * kPanel) : kPanel;  // rows in this panel
  tm = panel * kPanel + i % pm;
  tn = i / pm;
}
__device__ __forceinline__ void tile_of(int b, int G, int nt, int mt, int &tm, int &tn) {
  tile_coords(xcd_rank(b, G), nt, mt, tm, tn);
}

// Split schedule of a launch over nt x mtiles tiles:
//   P == 1            whole tiles in the XCD-aware order of tile_of;
//   P > 1, W == 0     every tile split along K into P pieces (launches of
//                     few tiles): units go (row block, piece, column tile)
//                     over XCD-contiguous ranks, so the row blocks and pieces
//                     of one column tile run on one XCD at once and share
//                     its weight and activation lines in that L2;
//   P > 1, W > 0      tail split: workgroups [0, W) take logical tiles
//                     [0, W) whole -- the full rounds of workgroup slots --
//                     and the rest, the last partial round's tiles, are cut
//                     into P pieces each, so that round ends after 1/P of a
//                     tile's time instead of a whole one.  Workgroups are
//                     dispatched in index order, so the pieces go last.
// sidx: the split index of the tile (its partials and arrival counter), or
// -1 for a whole tile.
__device__ __forceinline__ void sched_tile(int nt, int mtiles, int P, int W, int &tm, int &tn, int &piece, int &sidx) {
  const int b = blockIdx.x, G = gridDim.x;
  piece = 0;
  sidx = -1;
  if (P == 1) {
    tile_of(b, G, nt, mtiles, tm, tn);
  } else if (W == 0) {
    const int u = xcd_rank(b, G);
    tm = u % mtiles;
    piece = (u / mtiles) % P;
    tn = u / (mtiles * P);
    sidx = tn * mtiles + tm;
  } else if (b < W) {
    tile_of(b, W, nt, mtiles, tm, tn);
  } else {
    const int u = xcd_rank(b - W, G - W);  // the pieces of one tile on one XCD
    piece = u % P;
    sidx = u / P;
    tile_coords(W + sidx, nt, mtiles, tm, tn);
  }
}

// SwiGLU epilogue (w.pair > 0, fused gate_up weight with gate rows [0, I)
// and up rows [I, 2I), I = 16 * pair).  A column tile of SW strips covers
// output columns of SW/2 strips: waves 0-1 multiply gate strips
// j0 .. j0 + SW/2 - 1 and waves 2-3 the up strips pair + j0 .. of the same
// outputs, with identical register layouts, so an up wave's value v of lane
// l belongs to the gate wave (wave - 2)'s value v of lane l.  Each wave owns
// SW/4 consecutive strips; `ps0` is its first physical strip and strips at
// or past `slim` read zeros.
template <int SW>
__device__ __forceinline__ void swiglu_strips(const WeightView &w, int tn, int wave, int &ps0, int &slim, int &j0) {
  const int pair = (int)w.pair;
  j0 = tn * (SW / 2) + (wave & 1) * (SW / 4);
  ps0 = wave < 2 ? j0 : pair + j0;
  slim = wave < 2 ? pair : 2 * pair;
}

// Hand 16 values per lane from the up waves (2, 3) to the gate waves (0, 1)
// through LDS (8 KB at `xch`).  Every wave calls it; the first barrier also
// ends the k loop's reads of the staging buffers.
__device__ __forceinline__ void swiglu_exchange(float *xch, int wave, int lane, const float (&up)[16], float (&got)[16]) {
  __syncthreads();
  if (wave >= 2)
#pragma unroll
    for (int v = 0; v < 16; ++v) xch[((wave - 2) * 16 + v) * 64 + lane] = up[v];
  __syncthreads();
  if (wave < 2)
#pragma unroll
    for (int v = 0; v < 16; ++v) got[v] = xch[(wave * 16 + v) * 64 + lane];
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
template <int FMT, int ACT, int MS, int NS, bool SWI>
__global__ __launch_bounds__(256) void k_gemm(GemmParams p) {
  typedef GemmShape<FMT, ACT> S;
  typedef FmtTraits<FMT> T;
  constexpr int KS = S::KS, BY = ActTraits<ACT>::BYTES;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];  // [2][PARTS][ROWS][STRIDE] bf16
  const WeightView &w = p.w;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r = lane & 15;
  int tm, tn;
  const int nt = SWI ? (int)((w.pair + 2 * NS - 1) / (2 * NS)) : (int)((w.n_strips + 4 * NS - 1) / (4 * NS));
  tile_of(blockIdx.x, gridDim.x, nt, (int)((p.M + S::ROWS - 1) / S::ROWS), tm, tn);
  const int m0 = tm * S::ROWS;
  int s0 = tn * (4 * NS) + wave * NS, slim = (int)w.n_strips, j0 = 0;
  if constexpr (SWI) swiglu_strips<4 * NS>(w, tn, wave, s0, slim, j0);
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
  else if constexpr (FMT == DIALQ_FORMAT_Q6_K)
    ra = make_rsrc(w.aux, (uint32_t)(total * 288));
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
        const bool valid = st < nstage && c < kc && sn < slim;
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
      for (int n = 0; n < NS; ++n) o[n] = make_bops<FMT, ActTraits<ACT>::F16OP>(slot[j][n]);
      // refill this chunk's ring slot with stage st+2 as soon as it is unpacked
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        const int c = (st + 2) * KS + j, sn = s0 + n;
        const bool valid = st + 2 < nstage && c < kc && sn < slim;
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
              for (int n = 0; n < NS; ++n) acc[ms][n] = mfma_op<ACT>(xa, o[n].b[t], acc[ms][n]);
            }
      } else {
        // Q6_K walks its 8 slices in two halves, so only 4 activation
        // operands per row group are live next to the weight operands
        constexpr int NH = FMT == DIALQ_FORMAT_Q6_K ? 2 : 1, NXH = T::NX / NH;
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
          for (int ms = 0; ms < MS; ++ms) {
            XOp<ACT> xo[NXH];
#pragma unroll
            for (int tt = 0; tt < NXH; ++tt) {
              const int t = hh * NXH + tt;
              const int row = ms * 16 + r, kk = j * S::CHUNK + T::xk(t, g);
              xo[tt].hi = *(const u32x4 *)(base + row * S::STRIDE + kk);
              if constexpr (S::PARTS == 2) xo[tt].lo = *(const u32x4 *)(base + (S::ROWS + row) * S::STRIDE + kk);
            }
#pragma unroll
            for (int n = 0; n < NS; ++n) {
              if constexpr (NH == 1) bops_mac<FMT, ACT>(o[n], xo, acc[ms][n]);
              else if (hh == 0) bops_mac<FMT, ACT, 0, NXH>(o[n], xo, acc[ms][n]);
              else bops_mac<FMT, ACT, NXH, NXH>(o[n], xo, acc[ms][n]);
            }
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

  // lane (g, r) holds rows 16ms + 4g + i of column 16(s0 + n) + r
  if constexpr (SWI) {
    // y[m, j] = silu(gate) * up; the NS tiles of one 16-row group per exchange
    static_assert(NS * 4 <= 16, "one exchange holds 16 values per lane");
    const int64_t I = w.pair * 16;
    float *xch = (float *)lds;
    float scale[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const int64_t col = (int64_t)(s0 + n) * 16 + r;
      scale[n] = col < w.N ? epilogue_scale<FMT>(w, col) : 0.0f;
    }
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      float mine[16], up[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) mine[v] = v < NS * 4 ? acc[ms][v / 4][v % 4] * scale[v / 4] : 0.0f;
      swiglu_exchange(xch, wave, lane, mine, up);
      if (wave < 2) {
        const int64_t rb = m0 + ms * 16 + g * 4;
#pragma unroll
        for (int n = 0; n < NS; ++n) {
          const int64_t j = (int64_t)(j0 + n) * 16 + r;
          if (j >= I) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (rb + i < p.M) store_out(p.y, (rb + i) * out_ld(w) + j, p.y_dtype, silu_mul(mine[n * 4 + i], up[n * 4 + i]));
        }
      }
    }
    return;
  }
  const bool full = m0 + S::ROWS <= p.M;
  const int64_t ldy = out_ld(w);
  auto body = [&](auto yd, auto chk) __attribute__((always_inline)) {
    typedef decltype(yd) Y;
    constexpr bool CHK = decltype(chk)::value;  // row checks only for the ragged last row tile
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const int64_t col = (int64_t)(s0 + n) * 16 + r;
      if (col >= w.N) continue;
      const float scale = epilogue_scale<FMT>(w, col);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        const int64_t rb = m0 + ms * 16 + g * 4;
        typename Y::T *py = (typename Y::T *)p.y + rb * ldy + col;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!CHK || rb + i < p.M) py[i * ldy] = Y::conv(acc[ms][n][i] * scale);
      }
    }
  };
  with_y_dtype(p.y_dtype, [&](auto yd) __attribute__((always_inline)) {
    if (full) body(yd, std::false_type{});
    else body(yd, std::true_type{});
  });
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
template <int ACT>
__device__ __forceinline__ f32x16 mfma32_op(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (ActTraits<ACT>::F16OP)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else return mfma32(a, b, c);
}

// Split-K fixup of a 32x32-kernel tile t: each of its P pieces publishes
// its partial (agent-scope relaxed stores, complete before the count); the
// last to arrive adds the P partials in piece order -- the same order
// whichever piece is last, so the result is deterministic -- into `acc`,
// re-arms the tile's counter and returns true; the others return false.
// `flag`: an LDS int the staging buffers do not overlap.
template <int MT, int NQ>
__device__ __forceinline__ bool split_fixup(const GemmParams &p, f32x16 (&acc)[MT][NQ], int t, int piece, int *flag) {
  constexpr int NV = MT * NQ * 16;
  const int tid = threadIdx.x, P = p.P;
  float *mine = p.part + ((size_t)t * P + piece) * (NV * 256);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        __hip_atomic_store(&mine[((mt * NQ + q) * 16 + v) * 256 + tid], acc[mt][q][v], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) *flag = __hip_atomic_fetch_add(&p.cnt[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == P - 1;
  __syncthreads();
  if (!*flag) return false;
  // all P partials (this piece's too, read back from L2) in piece order,
  // one piece's values in flight per round trip
  const rsrc_t rp = make_rsrc(p.part + (size_t)t * P * (NV * 256), (uint32_t)((size_t)P * NV * 256 * 4));
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][q][v] = 0.0f;
  for (int u = 0; u < P; ++u) {
    float pv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
      pv[i] = __uint_as_float(
          (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rp, (int)(((u * NV + i) * 256 + tid) * 4), 0, kSC1));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[mt][q][v] += pv[(mt * NQ + q) * 16 + v];
  }
  if (tid == 0) __hip_atomic_store(&p.cnt[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

template <int FMT, int ACT, int MT, int KS, int OCC, bool SWI>
__global__ __launch_bounds__(256, OCC) void k_gemm32(GemmParams p) {
  constexpr int CHUNK = 64, SK = KS * CHUNK, STEPS = SK / 16;
  constexpr int PARTS = ActTraits<ACT>::PARTS, BY = ActTraits<ACT>::BYTES;
  constexpr int ROWS = 32 * MT, STRIDE = SK + 8, BUF = PARTS * ROWS * STRIDE;
  constexpr int NQ = 2, PIECES = ROWS * SK / 8 / 256;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];  // [2][PARTS][ROWS][STRIDE] bf16
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, r = lane & 15, sub = (lane >> 4) & 1;
  int tm, tn, piece, sidx;
  const bool grp = !SWI && p.g.nm > 1;
  const int nt = grp ? p.g.tbase[p.g.nm] : SWI ? (int)((p.w.pair + 7) / 8) : (int)((p.w.n_strips + 15) / 16);
  const int mtiles = (int)((p.M + ROWS - 1) / ROWS);
  sched_tile(nt, mtiles, p.P, p.W, tm, tn, piece, sidx);
  if (tm >= mtiles || tn >= nt) return;  // a grid larger than the tiles (never planned)
  const int P = sidx < 0 ? 1 : p.P;  // pieces of this workgroup's tile
  const int jm = grp ? group_member(p.g, tn) : 0;
  const WeightView &w = grp ? p.g.wm[jm] : p.w;
  void *const yout = grp ? p.g.ym[jm] : p.y;
  if (grp) tn -= p.g.tbase[jm];
  const int m0 = tm * ROWS;
  int s0 = tn * 16 + wave * 4, slim = (int)w.n_strips, j0 = 0;
  if constexpr (SWI) swiglu_strips<16>(w, tn, wave, s0, slim, j0);
  const int K = (int)w.K;
  // this workgroup's chunks [c0, c1) (all of them unless the tile is split)
  const int c0 = (int)((int64_t)piece * w.k_chunks / P), c1 = (int)((int64_t)(piece + 1) * w.k_chunks / P);
  const int kc = c1 - c0;
  const int kend = (c1 * CHUNK < K) ? c1 * CHUNK : K;  // activations past the piece read as zeros
  const int nstage = (kc + KS - 1) / KS;
  const int64_t total = w.n_strips * w.k_chunks;
  const rsrc_t rt = make_rsrc(w.tiles, (uint32_t)(total * 1024));
  const int mrows = (int)((p.M - m0) < ROWS ? (p.M - m0) : ROWS);
  const rsrc_t rx = make_rsrc((const uint8_t *)p.x + (int64_t)m0 * K * BY, (uint32_t)((int64_t)mrows * K * BY));

  // Per-lane load bases, computed once: the loop adds a uniform stage offset
  // and compares it with a per-lane limit, so it needs no index arithmetic
  // and no reload of the weight view.  An activation piece is live while its
  // k is below kend (which also ends it past the last stage).
  XRaw<ACT> apre[PIECES];
  uint32_t abase[PIECES];
  int alim[PIECES];
#pragma unroll
  for (int q = 0; q < PIECES; ++q) {
    const int pc = tid + q * 256, row = pc / (SK / 8), kk = (pc % (SK / 8)) * 8;
    abase[q] = (uint32_t)((row * K + c0 * CHUNK + kk) * BY);
    alim[q] = kend - c0 * CHUNK - kk;
  }
  auto fetch_a = [&](int st) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q)
      apre[q] = xraw_load<ACT>(rx, st * SK < alim[q] ? abase[q] + (uint32_t)(st * SK * BY) : kOOB);
  };
  auto store_a = [&](int buf) {
    uint16_t *base = lds + buf * BUF;
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int pc = tid + q * 256, row = pc / (SK / 8), kk = (pc % (SK / 8)) * 8;
      const XOp<ACT> o = xraw_to_op<ACT>(apre[q]);
      *(u32x4 *)(base + row * STRIDE + kk) = o.hi;
      if constexpr (PARTS == 2) *(u32x4 *)(base + (ROWS + row) * STRIDE + kk) = o.lo;
    }
  };
  // weight bytes of (stage st, 16-k step j, column tile q) for this lane:
  // bbase[q] + the chunk's offset within the piece; a strip past the weight
  // keeps kOOB, which stays out of range under any in-piece offset
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  uint32_t bbase[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int strip = s0 + 2 * q + sub;
    bbase[q] = strip < slim ? ((uint32_t)strip * (uint32_t)w.k_chunks + (uint32_t)c0) * 1024u +
                                  (uint32_t)(r * 16 + 8 * h)
                            : kOOB;
  }
  auto bload = [&](int st, int j, int q) -> u32x2 {
    const int cc = st * KS + j / 4;  // chunk within the piece (uniform)
    const uint32_t off = cc < kc ? bbase[q] + (uint32_t)(cc * 1024 + (j % 4) * 256) : kOOB;
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

  // Prologue in the steady state's load order (activations of stage st+1,
  // then weights of stage st+1), so the first stage waits like every other.
  fetch_b(wb[0], 0);
  fetch_a(0);
  store_a(0);
  fetch_a(1);
  __builtin_amdgcn_sched_barrier(0);
  fetch_b(wb[1], 1);
  __builtin_amdgcn_sched_barrier(0);

  auto bconv = [&](u32x2 v) -> u32x4 {
    constexpr bool F16 = ActTraits<ACT>::F16OP;
    if constexpr (FMT == DIALQ_FORMAT_W8A16) return F16 ? i8x8_to_f16(v[0], v[1]) : i8x8_to_bf16(v[0], v[1]);
    else return F16 ? e4m3x8_to_f16(v[0], v[1]) : e4m3x8_to_bf16(v[0], v[1]);
  };
  // B operands of a stage's first 16-k step, converted at the end of the
  // stage before: after the barrier the first MFMAs wait only for their
  // activation reads, so the two waves a barrier lines up on a SIMD do not
  // both spend the stage's start on conversions while the MFMA pipe idles.
  u32x4 b0[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) b0[q] = bconv(wb[0][0][q]);
  __builtin_amdgcn_sched_barrier(0);

  auto stage = [&](u32x2 (&slot)[STEPS][NQ], u32x2 (&nxt)[STEPS][NQ], int st) {
    __syncthreads();  // buffer st&1 written; buffer (st+1)&1 no longer read
    const uint16_t *base = lds + (st & 1) * BUF;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
      u32x4 b[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        b[q] = j == 0 ? b0[q] : bconv(slot[j][q]);
        slot[j][q] = bload(st + 2, j, q);  // refill with stage st+2
      }
#pragma unroll
      for (int part = 0; part < PARTS; ++part)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = mt * 32 + (lane & 31), kk = j * 16 + 8 * h;
          const u32x4 a = *(const u32x4 *)(base + (part * ROWS + row) * STRIDE + kk);
#pragma unroll
          for (int q = 0; q < NQ; ++q) acc[mt][q] = mfma32_op<ACT>(a, b[q], acc[mt][q]);
        }
      if (j == 0) {
        // the next stage's activations into the buffer the barrier freed,
        // behind this step's MFMAs; then the loads of stage st+2
        __builtin_amdgcn_sched_barrier(0);
        store_a((st + 1) & 1);
        fetch_a(st + 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) b0[q] = bconv(nxt[0][q]);
    __builtin_amdgcn_sched_barrier(0);
  };
  int st = 0;
  for (; st + 1 < nstage; st += 2) {
    stage(wb[0], wb[1], st);
    stage(wb[1], wb[0], st + 1);
  }
  if (st < nstage) stage(wb[0], wb[1], st);

  if (sidx >= 0 && !split_fixup<MT, NQ>(p, acc, sidx, piece, (int *)(lds + 2 * BUF))) return;

  if constexpr (SWI) {
    // y[m, j] = silu(gate) * up, one 32x32 tile per exchange
    const int64_t I = w.pair * 16;
    float *xch = (float *)lds;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t col = (int64_t)(s0 + 2 * q) * 16 + (lane & 31);  // weight row of this lane
      const int64_t j = (int64_t)(j0 + 2 * q) * 16 + (lane & 31);     // output column
      const float scale = col < w.N ? w.row_scale[col] : 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float mine[16], up[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) mine[v] = acc[mt][q][v] * scale;
        swiglu_exchange(xch, wave, lane, mine, up);
        if (wave < 2 && j < I) {
          const int64_t rb = m0 + mt * 32 + 4 * h;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t row = rb + 8 * (v / 4) + (v % 4);
            if (row < p.M) store_out(yout, row * out_ld(w) + j, p.y_dtype, silu_mul(mine[v], up[v]));
          }
        }
      }
    }
    return;
  }
  const bool full = m0 + ROWS <= p.M;
  const int64_t ldy = out_ld(w);
  auto body = [&](auto yd, auto chk) __attribute__((always_inline)) {
    typedef decltype(yd) Y;
    constexpr bool CHK = decltype(chk)::value;  // row checks only for the ragged last row tile
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t col = (int64_t)(s0 + 2 * q) * 16 + (lane & 31);
      if (col >= w.N) continue;
      const float scale = w.row_scale[col];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int64_t rb = m0 + mt * 32 + 4 * h;
        typename Y::T *py = (typename Y::T *)yout + rb * ldy + col;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rr = 8 * (v / 4) + (v % 4);
          if (!CHK || rb + rr < p.M) py[rr * ldy] = Y::conv(acc[mt][q][v] * scale);
        }
      }
    }
  };
  with_y_dtype(p.y_dtype, [&](auto yd) __attribute__((always_inline)) {
    if (full) body(yd, std::false_type{});
    else body(yd, std::true_type{});
  });
}

// ---------------------------------------------------------------------------
// GGUF prefill (Q4_K, Q8_0) on v_mfma_f32_32x32x16 with dequantized weight
// operands.  The weight-only k_gemm keeps these exact (codes as exact bf16,
// block scales applied to f32 partials; Q4_K with one extra MFMA per 32-k
// slice for its min term), which leaves it bound by VALU.  Prefill instead
// takes each weight as the value DIAL's GGUF prefill multiplies by -- the
// format's dequantized value in f32 (Q4_K d*sc*q - dmin*m, Q8_0 d*q) rounded
// to f16, the weight build_worker_gguf_fp16_prefill_linear dequantizes once
// (qwen3_vl/worker_gguf.rs:426-455, candle's to_float) -- against f16
// activations (the GGUF worker's dtype), one MFMA per 16-k step.  bf16
// activations are made f16 rows in range first (k_x_f16_rows) or, where no
// room is left for that copy, take the f32 weight as a bf16 hi + lo pair
// (two MFMAs, 2^-17 relative), since one bf16 rounding of the weight alone
// (2^-9) would dominate the product's error.
//
// Layout as k_gemm32: a 256-thread workgroup computes a (32*MT) x 256 tile;
// wave v owns 32-column MFMA tiles q = 0, 1 (strips s0 + 2q, s0 + 2q + 1;
// lane l: column l % 32, k group h = l / 32).  A stage is 64 k; step j of
// a stage (16 k) reads lane group g = 2(j % 2) + h of the resident tile.
//   Q4_K: a stage is quarter i of a 256-k chunk: k = 64i + 8g + j' (low
//         nibbles, sub-block 2i) and 64i + 32 + 8g + j' (high nibbles,
//         sub-block 2i + 1) sit in byte 8i + j' of tile lane r + 16g: steps
//         0-1 take the low nibbles, 2-3 the high ones -- two 8-byte loads
//         per column tile, plus the row's 16-byte block header.
//   Q8_0: a stage is one 64-k tile: block b = j / 2 sits in bytes 8b..8b+7
//         of lane r + 16g -- two 16-byte loads per column tile, plus the
//         row's two f16 block scales.
// ---------------------------------------------------------------------------
template <int ACT>
__device__ __forceinline__ void kq_pack(const float (&wv)[8], u32x4 &hi, u32x4 &lo) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (ACT == kActF16N) {
      const h2 v = {(_Float16)wv[2 * i], (_Float16)wv[2 * i + 1]};
      hi[i] = __builtin_bit_cast(uint32_t, v);
    } else {
      const b2 v = {(__bf16)wv[2 * i], (__bf16)wv[2 * i + 1]};
      const uint32_t hb = __builtin_bit_cast(uint32_t, v);
      const b2 u = {(__bf16)(wv[2 * i] - __uint_as_float(hb << 16)),
                    (__bf16)(wv[2 * i + 1] - __uint_as_float(hb & 0xffff0000u))};
      hi[i] = hb;
      lo[i] = __builtin_bit_cast(uint32_t, u);
    }
  }
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int FMT>
struct KqFmt;

template <>
struct KqFmt<DIALQ_FORMAT_Q4_K> {
  static constexpr int CHUNK = 256, TILE = 2048, AUX = 256;
  struct Slot {
    u32x2 c[2];  // lane groups h and 2 + h: bytes 8i..8i+7
    u32x4 hd;    // block header {d, dmin, scales[12]}
  };
  struct Sc {
    float s1[2], s2[2];  // d*sc and dmin*m of sub-blocks 2i, 2i + 1
  };
  static __device__ __forceinline__ void fetch(Slot &sl, rsrc_t rt, rsrc_t ra, uint32_t tile, int i, bool valid, int r,
                                               int h) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t off = tile * 2048u + (uint32_t)(i / 2) * 1024u + (uint32_t)(16 * (r + 16 * (2 * e + h)) + 8 * (i % 2));
      sl.c[e] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rt, valid ? (int)off : (int)kOOB, 0, 0));
    }
    sl.hd = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, valid ? (int)(tile * 256u + 16u * (uint32_t)r) : (int)kOOB, 0, 0));
  }
  // the 6-bit packing of candle's get_scale_min_k4; products exact in f32
  template <int I>
  static __device__ __forceinline__ Sc scales(const Slot &sl) {
    const u32x4 hd = sl.hd;
    const float d = f16_bits_to_f32(hd[0] & 0xffffu), dmin = f16_bits_to_f32(hd[0] >> 16);
    Sc o;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int j = 2 * I + e;
      uint32_t sc, mn;
      if (j < 4) {
        sc = (hd[1] >> (8 * j)) & 63u;
        mn = (hd[2] >> (8 * j)) & 63u;
      } else {
        const int jj = j - 4;
        const uint32_t b8 = (hd[3] >> (8 * jj)) & 0xffu;
        sc = (b8 & 0xfu) | (((hd[1] >> (8 * jj + 6)) & 3u) << 4);
        mn = (b8 >> 4) | (((hd[2] >> (8 * jj + 6)) & 3u) << 4);
      }
      o.s1[e] = d * (float)sc;
      o.s2[e] = dmin * (float)mn;
    }
    return o;
  }
  // f32 weights of step j: the high nibbles are taken in place (16q)
  // against s1 / 16 (exact)
  static __device__ __forceinline__ void weights(const Slot &sl, const Sc &sc, int j, float (&wv)[8]) {
    const bool high = j >= 2;
    const uint32_t m = high ? 0xf0f0f0f0u : 0x0f0f0f0fu;
    const float s1 = high ? sc.s1[1] * 0.0625f : sc.s1[0], s2 = high ? sc.s2[1] : sc.s2[0];
    uint32_t x[2] = {sl.c[j & 1][0] & m, sl.c[j & 1][1] & m};
    // opaque to the optimizer: it would otherwise fold each byte's mask into
    // a bit-field extract and convert from byte 0 (two instructions per
    // value); this way one AND per four values and v_cvt_f32_ubyte0..3
    asm("" : "+v"(x[0]), "+v"(x[1]));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      wv[4 * i] = __builtin_fmaf(s1, (float)(x[i] & 0xffu), -s2);
      wv[4 * i + 1] = __builtin_fmaf(s1, (float)((x[i] >> 8) & 0xffu), -s2);
      wv[4 * i + 2] = __builtin_fmaf(s1, (float)((x[i] >> 16) & 0xffu), -s2);
      wv[4 * i + 3] = __builtin_fmaf(s1, (float)(x[i] >> 24), -s2);
    }
  }
};

template <>
struct KqFmt<DIALQ_FORMAT_Q8_0> {
  static constexpr int CHUNK = 64, TILE = 1024, AUX = 64;
  struct Slot {
    u32x4 c[2];  // lane groups h and 2 + h: blocks 0 (bytes 0-7) and 1 (8-15)
    uint32_t d;  // the row's f16 scales of blocks 0 and 1
  };
  struct Sc {
    float d[2];
  };
  static __device__ __forceinline__ void fetch(Slot &sl, rsrc_t rt, rsrc_t ra, uint32_t tile, int i, bool valid, int r,
                                               int h) {
    (void)i;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t off = tile * 1024u + (uint32_t)(16 * (r + 16 * (2 * e + h)));
      sl.c[e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rt, valid ? (int)off : (int)kOOB, 0, 0));
    }
    sl.d = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ra, valid ? (int)(tile * 64u + 4u * (uint32_t)r) : (int)kOOB,
                                                          0, 0);
  }
  template <int I>
  static __device__ __forceinline__ Sc scales(const Slot &sl) {
    Sc o;
    o.d[0] = f16_bits_to_f32(sl.d & 0xffffu);
    o.d[1] = f16_bits_to_f32(sl.d >> 16);
    return o;
  }
  // f32 weights d*q of step j (exact: 11 x 8 significant bits): the codes
  // are read as unsigned bytes q + 128 (sign bit flipped) and d*(q + 128) -
  // 128 d is one fused multiply-add
  static __device__ __forceinline__ void weights(const Slot &sl, const Sc &sc, int j, float (&wv)[8]) {
    const int b = j >> 1;
    const float d = sc.d[b], off = -128.0f * d;
    const uint32_t x[2] = {sl.c[j & 1][2 * b] ^ 0x80808080u, sl.c[j & 1][2 * b + 1] ^ 0x80808080u};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      wv[4 * i] = __builtin_fmaf(d, (float)(x[i] & 0xffu), off);
      wv[4 * i + 1] = __builtin_fmaf(d, (float)((x[i] >> 8) & 0xffu), off);
      wv[4 * i + 2] = __builtin_fmaf(d, (float)((x[i] >> 16) & 0xffu), off);
      wv[4 * i + 3] = __builtin_fmaf(d, (float)(x[i] >> 24), off);
    }
  }
};

template <>
struct KqFmt<DIALQ_FORMAT_Q6_K> {
  static constexpr int CHUNK = 256, TILE = 3072, AUX = 288;
  // Stage i of the chunk: 32-k slices 2i, 2i + 1 (t = 4hh + qd, hh = i / 2,
  // qd = 2(i % 2) + s / 2 for step s): the low nibble (i even) or high nibble
  // (i odd) of ql bytes 8(s / 2)..+7 in plane hh, with bits 2qd of the qh
  // bytes 8hh..8hh+7 (plane 2) on top; sub-block 4i + s is step s.
  struct Slot {
    u32x4 ql[2];   // lane groups h and 2 + h: plane hh, 16 bytes
    u32x2 qh[2];   // the same lanes: plane 2, bytes 8hh..8hh+7
    uint32_t sc;   // i8 scales of sub-blocks 4i..4i+3 of the lane's row
    uint32_t d;    // the row's f16 d
  };
  struct Sc {
    float s1[4];  // d * sc of the stage's four sub-blocks (exact)
  };
  static __device__ __forceinline__ void fetch(Slot &sl, rsrc_t rt, rsrc_t ra, uint32_t tile, int i, bool valid, int r,
                                               int h) {
    const uint32_t hh = (uint32_t)(i / 2);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t lo = tile * 3072u + 16u * (uint32_t)(r + 16 * (2 * e + h));
      sl.ql[e] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rt, valid ? (int)(lo + hh * 1024u) : (int)kOOB, 0, 0));
      sl.qh[e] = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(rt, valid ? (int)(lo + 2048u + 8u * hh) : (int)kOOB, 0, 0));
    }
    const uint32_t ab = tile * 288u;
    sl.sc = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ra, valid ? (int)(ab + 16u * (uint32_t)r + 4u * (uint32_t)i)
                                                                   : (int)kOOB, 0, 0);
    sl.d = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(ra, valid ? (int)(ab + 256u + 2u * (uint32_t)r) : (int)kOOB,
                                                          0, 0);
  }
  template <int I>
  static __device__ __forceinline__ Sc scales(const Slot &sl) {
    const float d = f16_bits_to_f32(sl.d & 0xffffu);
    Sc o;
#pragma unroll
    for (int s = 0; s < 4; ++s) o.s1[s] = d * sbyte_f32(sl.sc, s);
    return o;
  }
  // f32 weights d*sc*(q6 - 32) of step j, each a single rounding of the
  // exact value
  template <int I>
  static __device__ __forceinline__ void weights_i(const Slot &sl, const Sc &sc, int j, float (&wv)[8]) {
    constexpr int NIB = 4 * (I % 2);
    const int qd = 2 * (I % 2) + (j >> 1);
    const float s1 = sc.s1[j], off = -32.0f * s1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t v = ((sl.ql[j & 1][2 * (j >> 1) + i] >> NIB) & 0x0f0f0f0fu) |
                         (((sl.qh[j & 1][i] >> (2 * qd)) & 0x03030303u) << 4);
      wv[4 * i] = __builtin_fmaf(s1, (float)(v & 0xffu), off);
      wv[4 * i + 1] = __builtin_fmaf(s1, (float)((v >> 8) & 0xffu), off);
      wv[4 * i + 2] = __builtin_fmaf(s1, (float)((v >> 16) & 0xffu), off);
      wv[4 * i + 3] = __builtin_fmaf(s1, (float)(v >> 24), off);
    }
  }
};

template <int FMT, int ACT, int MT, int OCC, bool SWI>
__global__ __launch_bounds__(256, OCC) void k_gemm_kq(GemmParams p) {
  static_assert(ACT == DIALQ_BF16 || ACT == kActF16N, "bf16 or f16 activations");
  typedef KqFmt<FMT> F;
  constexpr int SPC = F::CHUNK / 64;  // stages per resident chunk
  constexpr bool HL = ACT == DIALQ_BF16;  // weight as bf16 hi + lo
  constexpr int SK = 64, BY = 2;
  constexpr int ROWS = 32 * MT, STRIDE = SK + 8, BUF = ROWS * STRIDE;
  constexpr int NQ = 2, PIECES = ROWS * SK / 8 / 256;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];  // [2][ROWS][STRIDE]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, r = lane & 15, sub = (lane >> 4) & 1;
  int tm, tn, piece, sidx;
  const bool grp = !SWI && p.g.nm > 1;
  const int nt = grp ? p.g.tbase[p.g.nm] : SWI ? (int)((p.w.pair + 7) / 8) : (int)((p.w.n_strips + 15) / 16);
  const int mtiles = (int)((p.M + ROWS - 1) / ROWS);
  sched_tile(nt, mtiles, p.P, p.W, tm, tn, piece, sidx);
  if (tm >= mtiles || tn >= nt) return;  // a grid larger than the tiles (never planned)
  const int P = sidx < 0 ? 1 : p.P;  // pieces of this workgroup's tile
  const int jm = grp ? group_member(p.g, tn) : 0;
  const WeightView &w = grp ? p.g.wm[jm] : p.w;
  void *const yout = grp ? p.g.ym[jm] : p.y;
  if (grp) tn -= p.g.tbase[jm];
  const int m0 = tm * ROWS;
  int s0 = tn * 16 + wave * 4, slim = (int)w.n_strips, j0 = 0;
  if constexpr (SWI) swiglu_strips<16>(w, tn, wave, s0, slim, j0);
  const int K = (int)w.K;
  // this workgroup's chunks [c0, c1): SPC stages each
  const int c0 = (int)((int64_t)piece * w.k_chunks / P), c1 = (int)((int64_t)(piece + 1) * w.k_chunks / P);
  const int nstage = SPC * (c1 - c0);
  const int kend = (c1 * F::CHUNK < K) ? c1 * F::CHUNK : K;
  const int64_t total = w.n_strips * w.k_chunks;
  const rsrc_t rt = make_rsrc(w.tiles, (uint32_t)(total * F::TILE));
  const rsrc_t ra = make_rsrc(w.aux, (uint32_t)(total * F::AUX));
  const int mrows = (int)((p.M - m0) < ROWS ? (p.M - m0) : ROWS);
  const rsrc_t rx = make_rsrc((const uint8_t *)p.x + (int64_t)m0 * K * BY, (uint32_t)((int64_t)mrows * K * BY));

  // Per-lane load bases, computed once (as in k_gemm32): the loop adds a
  // uniform stage offset, and an activation piece is live while its k is
  // below kend.
  XRaw<ACT> apre[PIECES];
  uint32_t abase[PIECES];
  int alim[PIECES];
#pragma unroll
  for (int q = 0; q < PIECES; ++q) {
    const int pc = tid + q * 256, row = pc / (SK / 8), kk = (pc % (SK / 8)) * 8;
    abase[q] = (uint32_t)((row * K + c0 * F::CHUNK + kk) * BY);
    alim[q] = kend - c0 * F::CHUNK - kk;
  }
  auto fetch_a = [&](int st) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q)
      apre[q] = xraw_load<ACT>(rx, st * SK < alim[q] ? abase[q] + (uint32_t)(st * SK * BY) : kOOB);
  };
  auto store_a = [&](int buf) {
    uint16_t *base = lds + buf * BUF;
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int pc = tid + q * 256, row = pc / (SK / 8), kk = (pc % (SK / 8)) * 8;
      *(u32x4 *)(base + row * STRIDE + kk) = apre[q].a;
    }
  };
  // stage st's codes and scales of column tile q, for this lane's weight row
  struct Slot {
    typename F::Slot q[NQ];
  };
  uint32_t tbase[NQ];  // tile index of this lane's strip at chunk c0
  bool slive[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int strip = s0 + 2 * q + sub;
    slive[q] = strip < slim;
    tbase[q] = (uint32_t)strip * (uint32_t)w.k_chunks + (uint32_t)c0;
  }
  auto fetch_b = [&](Slot &sl, int st) {
    const int i = st % SPC;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      F::fetch(sl.q[q], rt, ra, tbase[q] + (uint32_t)(st / SPC), i, st < nstage && slive[q], r, h);
  };

  f32x16 acc[MT][NQ];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][q][v] = 0.0f;

  Slot wb[2];
  fetch_b(wb[0], 0);
  fetch_a(0);
  store_a(0);
  fetch_a(1);
  __builtin_amdgcn_sched_barrier(0);
  fetch_b(wb[1], 1);
  __builtin_amdgcn_sched_barrier(0);

  // B operands of a stage's first 16-k step, built at the end of the stage
  // before (as in k_gemm32): after the barrier the first MFMAs wait only
  // for their activation reads.  Q8_0 only: its 27B layer at M = 2048 gains
  // 3 % (791-792 -> 812-817 TFLOP/s) while Q4_K's loses 2-4 % (its larger
  // per-step build then sits on the stage's critical tail), Q6_K's kernel
  // already holds 256 VGPRs (the early operands spill 136 bytes per lane)
  // and the bf16 hi + lo form would spill 12.
  constexpr bool PRE = FMT == DIALQ_FORMAT_Q8_0 && !HL;
  u32x4 b0h[NQ], b0l[NQ];
  auto first_ops = [&](const Slot &sl, auto quarter) {
    constexpr int I = decltype(quarter)::value;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const typename F::Sc sc = F::template scales<I>(sl.q[q]);
      float wv[8];
      if constexpr (FMT == DIALQ_FORMAT_Q6_K) F::template weights_i<I>(sl.q[q], sc, 0, wv);
      else F::weights(sl.q[q], sc, 0, wv);
      kq_pack<ACT>(wv, b0h[q], b0l[q]);
    }
  };
  if constexpr (PRE) first_ops(wb[0], std::integral_constant<int, 0>{});
  __builtin_amdgcn_sched_barrier(0);

  auto stage = [&](Slot &sl, const Slot &nxt, int st, auto quarter, auto nquarter) {
    constexpr int I = decltype(quarter)::value;
    __syncthreads();  // buffer st&1 written; buffer (st+1)&1 no longer read
    if constexpr (!PRE) {
      store_a((st + 1) & 1);
      fetch_a(st + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    typename F::Sc sc[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) sc[q] = F::template scales<I>(sl.q[q]);
    const Slot cur = sl;
    fetch_b(sl, st + 2);  // refill with stage st + 2
    const uint16_t *base = lds + (st & 1) * BUF;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 bh[NQ], bl[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        if (PRE && j == 0) {
          bh[q] = b0h[q];
          bl[q] = b0l[q];
          continue;
        }
        float wv[8];
        if constexpr (FMT == DIALQ_FORMAT_Q6_K) F::template weights_i<I>(cur.q[q], sc[q], j, wv);
        else F::weights(cur.q[q], sc[q], j, wv);
        kq_pack<ACT>(wv, bh[q], bl[q]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 32 + (lane & 31), kk = j * 16 + 8 * h;
        const u32x4 a = *(const u32x4 *)(base + row * STRIDE + kk);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          acc[mt][q] = mfma32_op<ACT>(a, bh[q], acc[mt][q]);
          if constexpr (HL) acc[mt][q] = mfma32_op<ACT>(a, bl[q], acc[mt][q]);
        }
      }
      if (PRE && j == 0) {
        // the next stage's activations into the buffer the barrier freed,
        // behind this step's MFMAs; then the loads of stage st+2
        __builtin_amdgcn_sched_barrier(0);
        store_a((st + 1) & 1);
        fetch_a(st + 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (PRE) first_ops(nxt, nquarter);
    __builtin_amdgcn_sched_barrier(0);
  };
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;
  using Q2 = std::integral_constant<int, 2>;
  using Q3 = std::integral_constant<int, 3>;
  if constexpr (SPC == 4) {
    for (int st = 0; st < nstage; st += 4) {
      stage(wb[0], wb[1], st, Q0{}, Q1{});
      stage(wb[1], wb[0], st + 1, Q1{}, Q2{});
      stage(wb[0], wb[1], st + 2, Q2{}, Q3{});
      stage(wb[1], wb[0], st + 3, Q3{}, Q0{});
    }
  } else {
    int st = 0;
    for (; st + 1 < nstage; st += 2) {
      stage(wb[0], wb[1], st, Q0{}, Q0{});
      stage(wb[1], wb[0], st + 1, Q0{}, Q0{});
    }
    if (st < nstage) stage(wb[0], wb[1], st, Q0{}, Q0{});
  }

  if (sidx >= 0 && !split_fixup<MT, NQ>(p, acc, sidx, piece, (int *)(lds + 2 * BUF))) return;

  if constexpr (SWI) {
    const int64_t I = w.pair * 16;
    float *xch = (float *)lds;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t j = (int64_t)(j0 + 2 * q) * 16 + (lane & 31);  // output column
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float mine[16], up[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) mine[v] = acc[mt][q][v];
        swiglu_exchange(xch, wave, lane, mine, up);
        if (wave < 2 && j < I) {
          const int64_t rb = m0 + mt * 32 + 4 * h;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t row = rb + 8 * (v / 4) + (v % 4);
            if (row < p.M) {
              const float f = p.yrow ? p.yrow[row] : 1.0f;
              store_out(yout, row * out_ld(w) + j, p.y_dtype, silu_mul(mine[v] * f, up[v] * f));
            }
          }
        }
      }
    }
    return;
  }
  const bool full = m0 + ROWS <= p.M;
  const int64_t ldy = out_ld(w);
  auto body = [&](auto yd, auto chk) __attribute__((always_inline)) {
    typedef decltype(yd) Y;
    constexpr bool CHK = decltype(chk)::value;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t col = (int64_t)(s0 + 2 * q) * 16 + (lane & 31);
      if (col >= w.N) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int64_t rb = m0 + mt * 32 + 4 * h;
        typename Y::T *py = (typename Y::T *)yout + rb * ldy + col;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rr = 8 * (v / 4) + (v % 4);
          if (!CHK || rb + rr < p.M) py[rr * ldy] = Y::conv(p.yrow ? acc[mt][q][v] * p.yrow[rb + rr] : acc[mt][q][v]);
        }
      }
    }
  };
  with_y_dtype(p.y_dtype, [&](auto yd) __attribute__((always_inline)) {
    if (full) body(yd, std::false_type{});
    else body(yd, std::true_type{});
  });
}

// Launch plan of the 32x32 kernel.  Two shapes: 64-row tiles with one 64-k
// chunk per stage (GEMM32_MT, GEMM32_KS) for prefill, and for 17..96 rows
// 32-row tiles with two chunks per stage: those launches have few tiles, so
// each workgroup's weight stream is latency bound, and half the accumulators
// with twice the weight bytes per stage keep more of it in flight (measured
// on the 27B shapes at 24..96 rows: 1.2-1.6x faster than 64-row tiles).
// A launch with few tiles also leaves CUs idle; it splits every tile along K
// into P pieces (split-K), at least kGemm32MinChunks chunks each.  A piece
// writes a rows x 256 f32 partial tile and the last one reads them all
// back, traffic worth spending only while the tiles are far fewer than the
// CUs: small-row launches split while tiles fill at most half the workgroup
// slots (<= 8 pieces), prefill launches only below CUs / 2 tiles
// (<= 4 pieces; the 17408-row gate at 128 rows, 136 tiles, is faster whole),
// and never past kGemm32MaxPartBytes of partials.
constexpr int64_t kGemm32SmallRows = 96;
// W8A16 / FP8_ROW from this many rows: 128-row tiles at 2 workgroups per CU
// (gate 17408x5120 at M = 2048: 961 against 883 TFLOP/s with 64-row tiles at
// 3 per CU; at M = 1024 the 544 tiles of 128 rows leave most of a second
// round of 512 slots idle and lose, 763 against 842)
constexpr int64_t kGemm32TallRows = 2048;
constexpr int kGemm32MinChunks = 20;  // 64-k steps per split-K piece, at least
constexpr size_t kGemm32MaxPartBytes = (size_t)31 << 20;
// Tail split of a launch of `tiles` tiles over `slots` resident workgroup
// slots whose last round is at most half full (the 27B gate 17408x5120 at
// M = 2048 in 128-row tiles: 1088 tiles, two rounds of 512 and 64 left):
// the full rounds' tiles stay whole and the last round's are cut along K
// into P pieces, at most kTailMaxPieces, each at least kTailMinChunks
// chunks, their partial tiles within `budget` bytes.  The tail then takes
// about 1/P of a tile's time plus the last piece's read-back of the
// partials, instead of a whole tile's time with most slots idle.
constexpr int kTailMaxPieces = 8;
constexpr int kTailMinChunks = 4;
constexpr size_t kTailPartBytes = (size_t)32 << 20;  // default budget of the tail's partials

struct SplitPlan {
  int P = 1;           // pieces per split tile
  int64_t W = 0;       // tail split: tiles [0, W) whole (0: every tile split when P > 1)
  int64_t tiles = 0;
  size_t tile_part = 0;  // bytes of one piece's partial tile
  int64_t nsplit() const { return P > 1 ? (W > 0 ? tiles - W : tiles) : 0; }
  size_t part_bytes() const { return (size_t)(nsplit() * P) * tile_part; }
  int64_t grid() const { return P > 1 ? W + nsplit() * P : tiles; }
};

static void tail_split(SplitPlan &s, int64_t slots, int64_t kc, size_t budget, int max_pieces = kTailMaxPieces) {
  if (s.P > 1 || s.tiles <= slots) return;
  const int64_t tail = s.tiles % slots;
  if (tail == 0 || 2 * tail > slots) return;
  int64_t P = slots / tail;
  if (P > max_pieces) P = max_pieces;
  if (P > kc / kTailMinChunks) P = kc / kTailMinChunks;
  while (P > 1 && (size_t)(tail * P) * s.tile_part > budget) --P;
  if (P < 2) return;
  s.P = (int)P;
  s.W = s.tiles - tail;
}

struct Gemm32Plan : SplitPlan {
  int mt, ks;
};
// 256-column tiles of a weight (pairs of gate / up strip groups for SwiGLU).
static int64_t gemm32_col_tiles(const WeightView &w) { return w.pair ? (w.pair + 7) / 8 : (w.n_strips + 15) / 16; }

// nt: column tiles of the launch (all members of a grouped one); budget:
// bytes allowed for a tail split's partials.
static Gemm32Plan gemm32_plan(int64_t M, const WeightView &w, int64_t nt, size_t budget) {
  Gemm32Plan g;
  // Launches of very few 128-row tiles (the 27B k / v at 256-512 rows: 8-16
  // tiles) take the small-row plan too -- 32-row tiles split along K -- so
  // that more than a handful of CUs work: W8A16 k / v at M = 256 23.7 ->
  // 19 us, the W8A16 layer at M = 512 597 -> 670 TFLOP/s (down 200 -> 152
  // us), Q4_K k / v at M = 256 59 -> 33 us.  The GGUF kernel dequantizes its
  // weight tile once per 32 rows there, so it takes this plan only below
  // CUs / 8 tiles (at 40-96 tiles its M = 512 layer lost 29 %).
  const bool kq = w.fmt == DIALQ_FORMAT_Q4_K || w.fmt == DIALQ_FORMAT_Q8_0 || w.fmt == DIALQ_FORMAT_Q6_K;
  const bool small = M <= kGemm32SmallRows || nt * ((M + 127) / 128) * (kq ? 8 : 2) < device_cus();
  g.mt = small ? 1 : kq ? GEMMKQ_MT : M >= kGemm32TallRows ? 4 : GEMM32_MT;
  // 128-row tiles that fill less than one round of their slots but too many
  // to split along K (the 27B o and down projections at 2048 rows: 320
  // tiles on 512 slots) leave a CU in four with two tiles and the rest
  // with one; 64-row tiles at three per CU spread them more evenly (down
  // 5120x17408: 440 -> 402 us, o 164 -> 160; q and k / v unchanged or
  // worse, so not past the split-K range)
  if (!kq && g.mt == 4 && nt * ((M + 127) / 128) < 2 * device_cus() && nt * ((M + 127) / 128) * 2 >= device_cus())
    g.mt = GEMM32_MT;
  g.ks = small ? 2 : GEMM32_KS;  // byte formats; a Q4_K stage is one 64-k quarter chunk
  const int64_t rows = 32 * g.mt;
  g.tiles = nt * ((M + rows - 1) / rows);
  g.tile_part = (size_t)rows * 256 * sizeof(float);
  g.P = 1;
  const int64_t occ = kq ? GEMMKQ_OCC : g.mt == 4 ? 2 : GEMM32_OCC;
  const int64_t cus = device_cus(), slots = occ * cus;
  if (small ? g.tiles * 2 <= slots : g.tiles * 2 < cus) {
    const int64_t steps = w.k_chunks * (w.fmt == DIALQ_FORMAT_Q4_K || w.fmt == DIALQ_FORMAT_Q6_K ? 4 : 1);
    int64_t P = slots / g.tiles, cap = steps / kGemm32MinChunks;
    if (cap > (small ? 8 : 4)) cap = small ? 8 : 4;
    if (P > cap) P = cap;
    g.P = (int)(P < 1 ? 1 : P);
    while (g.P > 1 && g.part_bytes() > kGemm32MaxPartBytes) --g.P;
  }
  if (!small) tail_split(g, slots, w.k_chunks, budget);
  return g;
}

// The 32x32 kernels: W8A16 / FP8_ROW (k_gemm32) and Q4_K / Q8_0 / Q6_K with
// bf16 or f16 activations (k_gemm_kq; f32 activations keep the exact k_gemm).
static bool gemm32_applies(const WeightView &w, int x_dtype) {
  if (w.fmt == DIALQ_FORMAT_W8A16 || w.fmt == DIALQ_FORMAT_FP8_ROW) return w.n_strips * w.k_chunks * 1024 <= 0xffffffffLL;
  if (w.fmt == DIALQ_FORMAT_Q4_K)
    return x_dtype != DIALQ_F32 && w.n_strips * w.k_chunks * 2048 <= 0xffffffffLL;
  if (w.fmt == DIALQ_FORMAT_Q8_0)
    return x_dtype != DIALQ_F32 && w.n_strips * w.k_chunks * 1024 <= 0xffffffffLL;
  if (w.fmt == DIALQ_FORMAT_Q6_K)
    return x_dtype != DIALQ_F32 && w.n_strips * w.k_chunks * 3072 <= 0xffffffffLL;
  return false;
}

void gemm_workspace(int64_t M, const WeightView &w, int x_dtype, size_t &part_bytes, size_t &cnt_count, bool tail) {
  part_bytes = 0;
  cnt_count = 0;
  if (!gemm32_applies(w, x_dtype) || M <= 0) return;
  const Gemm32Plan g = gemm32_plan(M, w, gemm32_col_tiles(w), tail ? kTailPartBytes : 0);
  part_bytes = g.part_bytes();
  cnt_count = (size_t)g.nsplit();
}

// The member table of a grouped 32x32-kernel launch, or false where one does
// not apply (a member the 32x32 kernels do not take, mixed formats or K,
// SwiGLU, more than kGemmMaxGroup members).
static bool gemm_group_table(const WeightView *ws, void *const *ys, int n, int x_dtype, GemmGroup &g) {
  if (n < 2 || n > kGemmMaxGroup) return false;
  g.nm = n;
  g.tbase[0] = 0;
  for (int j = 0; j < n; ++j) {
    if (ws[j].fmt != ws[0].fmt || ws[j].K != ws[0].K || ws[j].pair || !gemm32_applies(ws[j], x_dtype)) return false;
    g.wm[j] = ws[j];
    g.ym[j] = ys ? ys[j] : nullptr;
    g.tbase[j + 1] = g.tbase[j] + (int)gemm32_col_tiles(ws[j]);
  }
  for (int j = n; j < kGemmMaxGroup; ++j) g.tbase[j + 1] = g.tbase[n];
  return true;
}

bool gemm_group_workspace(int64_t M, const WeightView *ws, int n, int x_dtype, size_t &part_bytes, size_t &cnt_count) {
  part_bytes = 0;
  cnt_count = 0;
  GemmGroup g;
  if (M <= 0 || !gemm_group_table(ws, nullptr, n, x_dtype, g)) return false;
  const Gemm32Plan pl = gemm32_plan(M, ws[0], g.tbase[n], kTailPartBytes);
  part_bytes = pl.part_bytes();
  cnt_count = (size_t)pl.nsplit();
  return true;
}

template <int FMT, int ACT, int MT>
static hipError_t gemm_kq_launch(const GemmParams &p, int64_t grid, hipStream_t st) {
  constexpr int BUF = 32 * MT * (64 + 8);
  static_assert(2 * BUF * 2 >= 8192, "the SwiGLU exchange reuses the staging LDS");
  const size_t lds_bytes = 2 * BUF * 2 + 16;  // two staging buffers and the split-K arrival flag
  if (p.w.pair) k_gemm_kq<FMT, ACT, MT, GEMMKQ_OCC, true><<<(unsigned)grid, 256, lds_bytes, st>>>(p);
  else k_gemm_kq<FMT, ACT, MT, GEMMKQ_OCC, false><<<(unsigned)grid, 256, lds_bytes, st>>>(p);
  return hipGetLastError();
}

template <int FMT, int ACT, int MT, int KS, int OCC = GEMM32_OCC>
static hipError_t gemm32_launch(const GemmParams &p, int64_t grid, hipStream_t st) {
  constexpr int BUF = ActTraits<ACT>::PARTS * 32 * MT * (KS * 64 + 8);
  static_assert(2 * BUF * 2 >= 8192, "the SwiGLU exchange reuses the staging LDS");
  const size_t lds_bytes = 2 * BUF * 2 + 16;  // two staging buffers and the split-K arrival flag
  if (p.w.pair) k_gemm32<FMT, ACT, MT, KS, OCC, true><<<(unsigned)grid, 256, lds_bytes, st>>>(p);
  else k_gemm32<FMT, ACT, MT, KS, OCC, false><<<(unsigned)grid, 256, lds_bytes, st>>>(p);
  return hipGetLastError();
}

// grp: the member table of a grouped launch (null: the single weight w).
template <int FMT, int ACT>
static hipError_t gemm_dispatch(const WeightView &w, const void *x, int64_t M, void *y, int y_dtype, float *part,
                                size_t part_bytes, int *cnt, size_t cnt_count, hipStream_t st,
                                const GemmGroup *grp = nullptr, const float *yrow = nullptr) {
  typedef GemmShape<FMT, ACT> S;
  if ((int64_t)S::ROWS * w.K * ActTraits<ACT>::BYTES > 0xffffffffLL) return hipErrorInvalidValue;
  constexpr bool BYTE = FMT == DIALQ_FORMAT_W8A16 || FMT == DIALQ_FORMAT_FP8_ROW;
  constexpr bool KQ = (FMT == DIALQ_FORMAT_Q4_K || FMT == DIALQ_FORMAT_Q8_0 || FMT == DIALQ_FORMAT_Q6_K) &&
                      (ACT == DIALQ_BF16 || ACT == kActF16N);
  if constexpr (BYTE || KQ) {
    if (gemm32_applies(w, ACT == DIALQ_F32 ? DIALQ_F32 : DIALQ_BF16)) {
      // the tail budget the workspace was sized with, or the buffer given
      const Gemm32Plan g = gemm32_plan(M, w, grp ? grp->tbase[grp->nm] : gemm32_col_tiles(w),
                                       part_bytes < kTailPartBytes ? part_bytes : kTailPartBytes);
      if (g.P > 1 && ((size_t)g.nsplit() > cnt_count || g.part_bytes() > part_bytes)) return hipErrorInvalidValue;
      if (g.grid() > 0x7fffffffLL) return hipErrorInvalidValue;
      GemmParams p{w, x, y, M, y_dtype, g.P, part, cnt};
      p.W = (int)g.W;
      if (grp) p.g = *grp;
      p.yrow = yrow;
      if (yrow && !KQ) return hipErrorInvalidValue;
      // the plan's tile height must be one this launcher instantiates: the
      // grid and the split indices were counted in its tiles
      if constexpr (KQ) {
        if (g.mt == 1) return gemm_kq_launch<FMT, ACT, 1>(p, g.grid(), st);
        if (g.mt != GEMMKQ_MT) return hipErrorInvalidValue;
        return gemm_kq_launch<FMT, ACT, GEMMKQ_MT>(p, g.grid(), st);
      } else {
        if (g.mt == 1) return gemm32_launch<FMT, ACT, 1, 2>(p, g.grid(), st);
        if (g.mt == 4) return gemm32_launch<FMT, ACT, 4, 1, 2>(p, g.grid(), st);
        if (g.mt != GEMM32_MT) return hipErrorInvalidValue;
        return gemm32_launch<FMT, ACT, GEMM32_MT, GEMM32_KS>(p, g.grid(), st);
      }
    }
  }
  if (grp) return hipErrorNotSupported;
  if (yrow) return hipErrorInvalidValue;
  static_assert(S::LDS_BYTES >= 8192, "the SwiGLU exchange reuses the staging LDS");
  const int64_t nt = w.pair ? (w.pair + 2 * S::NS - 1) / (2 * S::NS) : (w.n_strips + 4 * S::NS - 1) / (4 * S::NS);
  dim3 grid((unsigned)(nt * ((M + S::ROWS - 1) / S::ROWS)));
  GemmParams p{w, x, y, M, y_dtype};
  if (w.pair) k_gemm<FMT, ACT, S::MS, S::NS, true><<<grid, 256, S::LDS_BYTES, st>>>(p);
  else k_gemm<FMT, ACT, S::MS, S::NS, false><<<grid, 256, S::LDS_BYTES, st>>>(p);
  return hipGetLastError();
}

template <int FMT>
static hipError_t gemm_act(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y, int y_dtype,
                           float *part, size_t part_bytes, int *cnt, size_t cnt_count, hipStream_t st,
                           const GemmGroup *grp = nullptr, const float *yrow = nullptr) {
  switch (x_dtype) {
    case DIALQ_BF16:
      return gemm_dispatch<FMT, DIALQ_BF16>(w, x, M, y, y_dtype, part, part_bytes, cnt, cnt_count, st, grp, yrow);
    // f16 activations go to f16 MFMAs as they are, against f16 weight
    // operands; MXFP4's scaled codes need bf16's exponent range (hi / lo parts)
    case DIALQ_F16:
      return gemm_dispatch<FMT, FMT == DIALQ_FORMAT_MXFP4 ? DIALQ_F16 : kActF16N>(
          w, x, M, y, y_dtype, part, part_bytes, cnt, cnt_count, st, grp, yrow);
    case DIALQ_F32:
      return gemm_dispatch<FMT, DIALQ_F32>(w, x, M, y, y_dtype, part, part_bytes, cnt, cnt_count, st, grp, yrow);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_group(const WeightView *ws, void *const *ys, int n, const void *x, int x_dtype, int64_t M,
                             int y_dtype, float *part, size_t part_bytes, int *cnt, size_t cnt_count, hipStream_t st,
                             const float *yrow) {
  GemmGroup g;
  if (!gemm_group_table(ws, ys, n, x_dtype, g)) return hipErrorNotSupported;
  hipError_t r = hipErrorNotSupported;
  switch (ws[0].fmt) {
    case DIALQ_FORMAT_W8A16:
      r = gemm_act<DIALQ_FORMAT_W8A16>(ws[0], x, x_dtype, M, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st, &g,
                                       yrow);
      break;
    case DIALQ_FORMAT_FP8_ROW:
      r = gemm_act<DIALQ_FORMAT_FP8_ROW>(ws[0], x, x_dtype, M, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st,
                                         &g, yrow);
      break;
    case DIALQ_FORMAT_Q4_K:
      r = gemm_act<DIALQ_FORMAT_Q4_K>(ws[0], x, x_dtype, M, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st, &g,
                                      yrow);
      break;
    case DIALQ_FORMAT_Q8_0:
      r = gemm_act<DIALQ_FORMAT_Q8_0>(ws[0], x, x_dtype, M, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st, &g,
                                      yrow);
      break;
    case DIALQ_FORMAT_Q6_K:
      r = gemm_act<DIALQ_FORMAT_Q6_K>(ws[0], x, x_dtype, M, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st, &g,
                                      yrow);
      break;
  }
  if (r == hipSuccess) g_prefill_grouped_launches.fetch_add(1, std::memory_order_relaxed);
  return r;
}

int64_t gemm_grouped_launches() { return g_prefill_grouped_launches.load(std::memory_order_relaxed); }

hipError_t launch_gemm(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y, int y_dtype, float *part,
                       size_t part_bytes, int *cnt, size_t cnt_count, hipStream_t st, const float *yrow) {
#define DIALQ_GEMM_FMT(F) \
  case F: return gemm_act<F>(w, x, x_dtype, M, y, y_dtype, part, part_bytes, cnt, cnt_count, st, nullptr, yrow);
  switch (w.fmt) {
    DIALQ_GEMM_FMT(DIALQ_FORMAT_W8A16)
    DIALQ_GEMM_FMT(DIALQ_FORMAT_FP8_ROW)
    DIALQ_GEMM_FMT(DIALQ_FORMAT_Q8_0)
    DIALQ_GEMM_FMT(DIALQ_FORMAT_FP8_BLOCK)
    DIALQ_GEMM_FMT(DIALQ_FORMAT_NVFP4)
    DIALQ_GEMM_FMT(DIALQ_FORMAT_MXFP4)
    DIALQ_GEMM_FMT(DIALQ_FORMAT_Q4_K)
    DIALQ_GEMM_FMT(DIALQ_FORMAT_Q6_K)
  }
#undef DIALQ_GEMM_FMT
  return hipErrorInvalidValue;
}

// ===========================================================================
// Native low-precision prefill on v_mfma_scale_f32_32x32x64_f8f6f4.
//
// Activations are quantized first (per-token E4M3 with an f32 scale; per-32
// MXFP4 with E8M0 scales).  Measured issue rates of the scaled MFMAs on
// gfx950 (independent chains, no memory): 32x32x64 fp8 4.4 PFLOP/s and fp4
// 8.3 PFLOP/s, against 4.1 and 4.3 for the 16x16x128 form, so the 32x32 form
// is used for both.  Its operands: lane l holds row (A) / column (B) l % 32
// and the 32 k values 32*(l/32) .. +31 of a 64-k step, as 32 fp8 bytes or 32
// fp4 nibbles (low nibble first), with one E8M0 scale per lane for those 32
// values.  A resident weight tile (16 rows x 128 k) keeps row r, k block g at
// lane slot 16g + r, so a lane's B operand of step j is the slot
// 16(2j + l/32) + l%16 of the tile of strip 2q + (l/16)%2: one contiguous
// 32-byte (fp8) or 16-byte (fp4) buffer load.
//
// A 256-thread workgroup computes a (32*MT) x 256 tile of y: wave v owns the
// 64 columns of strips s0 .. s0+3 (s0 = 16*tn + 4v) as two 32-column MFMA
// tiles, and all 32*MT rows.  Activations of one 128-k chunk are staged in
// LDS (double-buffered, one barrier per chunk) and shared by the 4 waves;
// weights ride a two-chunk register ring, each slot refilled right after use.
//
// FP8_BLOCK's f32 128x128 weight scale ws_c is uniform over a wave (its 64
// columns lie in one 128-column block).  With ws_c = m_c * 2^e_c
// (m_c in [0.5, 1)) the accumulator R holds y / (xs[m] * mref): before chunk
// c it is multiplied by mref / m_c (skipped when equal) and mref = m_c, and
// the chunk's MFMAs carry 2^e_c as the weight's E8M0 scale, so
// y = xs[m] * mref * R = xs[m] * sum_c ws_c * (xq . wq)_c with no extra
// accumulator registers.  Chunks with ws_c == 0 contribute nothing and are
// skipped.  The e_c of a normal f32 scale lies in [-125, 128]; scales at or
// above 2^127 or below 2^-127 are clamped to the E8M0 range.
// ===========================================================================
struct NativeParams {
  WeightView w;
  const uint8_t *xq;  // FP8: [M, k_pad] E4M3; MXFP4: [M, k_pad/2] E2M1 codes
  const void *xs;     // FP8: [M] f32 per-token scale; MXFP4: [M, k_pad/32] E8M0
  int64_t M, k_pad;
  void *y;
  int y_dtype;
  // Split-K: P pieces per split tile (1: whole tiles, no partials); with
  // W > 0 only the tiles past the first W are split (sched_tile).
  int P;
  float *part;  // [split tiles][P][32 MT][256] partial tiles
  int *cnt;     // [split tiles] arrivals per split tile; zero between launches
  int W = 0;
  GemmGroup g;
};

template <bool FP8>
__device__ __forceinline__ f32x16 mfma_scaled32(i32x8 a, i32x8 b, f32x16 c, int sa, int sb) {
  if constexpr (FP8) return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
  else return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 4, 0, sa, 0, sb);
}

#ifndef NATIVE_MT_FP8
#define NATIVE_MT_FP8 2  // 32-row MFMA tiles per workgroup, FP8_BLOCK
#endif
#ifndef NATIVE_OCC_FP8
#define NATIVE_OCC_FP8 2  // workgroups per CU the FP8_BLOCK kernel is built for
#endif
#ifndef NATIVE_MT_FP4
#define NATIVE_MT_FP4 4
#endif
#ifndef NATIVE_OCC_FP4
#define NATIVE_OCC_FP4 2
#endif
#ifndef NATIVE_DEPTH_FP8
#define NATIVE_DEPTH_FP8 2  // chunks of weights and activations in flight per wave (register ring slots)
#endif
#ifndef NATIVE_DEPTH_FP4
#define NATIVE_DEPTH_FP4 2
#endif

// Fewest k chunks per piece of a split tile: a piece's partial (64 KB out,
// read back by the last piece) must be worth the extra parallelism; fp4
// chunks take half the MFMA time of fp8 ones (measured: MXFP4 k/v and q/o
// at 27B shapes are faster unsplit, the 136-chunk down projection split).
constexpr int native_min_chunks(int fmt) { return fmt == DIALQ_FORMAT_FP8_BLOCK ? 8 : 32; }

template <int FMT, int MT, int OCC, int DEPTH, bool SWI>
__global__ __launch_bounds__(256, OCC) void k_gemm_native(NativeParams p) {
  constexpr bool FP8 = FMT == DIALQ_FORMAT_FP8_BLOCK;
  constexpr int ROWB = FP8 ? 128 : 64;  // activation code bytes per row and chunk
  constexpr int STRIDE = ROWB + 16;     // padded LDS row: 16-lane b128 reads hit all 64 banks once
  constexpr int ROWS = 32 * MT, ABUF = ROWS * STRIDE;
  constexpr int NPIECE = ROWS * ROWB / 16, PIECES = (NPIECE + 255) / 256;
  static_assert(NPIECE % 256 == 0, "activation pieces must fill the workgroup");
  constexpr int ACC = MT * 2 * 16;  // accumulators per thread: MT x 2 tiles of 16
  constexpr int TILE = FP8 ? 2048 : 1024;  // resident tile bytes
  constexpr int BW = FP8 ? 2 : 1;          // 16-byte loads per lane and B operand
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * ABUF];
  __shared__ uint32_t lds_s[2][256];  // MXFP4: the 4 E8M0 scales of a row's chunk (rows < ROWS)
  __shared__ int lds_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, r = lane & 15, sub = (lane >> 4) & 1;
  const int kc = (int)p.w.k_chunks;
  const bool grp = !SWI && p.g.nm > 1;
  const int nt = grp ? p.g.tbase[p.g.nm] : SWI ? (int)((p.w.pair + 7) / 8) : (int)((p.w.n_strips + 15) / 16);
  const int mtiles = (int)((p.M + ROWS - 1) / ROWS);
  // One workgroup per tile or k piece of a tile (sched_tile).
  int tm, tn, piece, t;  // t: split index of the tile, -1 when whole
  sched_tile(nt, mtiles, p.P, p.W, tm, tn, piece, t);
  if (tm >= mtiles || tn >= nt) return;  // a grid larger than the tiles (never planned)
  const int P = t < 0 ? 1 : p.P;
  const int c0 = (int)((int64_t)piece * kc / P), c1 = (int)((int64_t)(piece + 1) * kc / P);
  const int jm = grp ? group_member(p.g, tn) : 0;
  const WeightView &w = grp ? p.g.wm[jm] : p.w;
  void *const yout = grp ? p.g.ym[jm] : p.y;
  if (grp) tn -= p.g.tbase[jm];
  const uint32_t pitch = (uint32_t)(FP8 ? p.k_pad : p.k_pad / 2);
  const rsrc_t rt = make_rsrc(w.tiles, (uint32_t)(w.n_strips * w.k_chunks * TILE));
  rsrc_t rb = rt;
  if constexpr (!FP8) rb = make_rsrc(w.aux, (uint32_t)(w.n_strips * w.k_chunks * 64));
  {
    const int m0 = tm * ROWS;
    int s0 = tn * 16 + wave * 4, slim = (int)w.n_strips, j0 = 0;
    if constexpr (SWI) swiglu_strips<16>(w, tn, wave, s0, slim, j0);
    const int mrows = (int)((p.M - m0) < ROWS ? (p.M - m0) : ROWS);
    const rsrc_t rx = make_rsrc(p.xq + (int64_t)m0 * pitch, (uint32_t)mrows * pitch);
    rsrc_t rs = rx;
    if constexpr (!FP8)
      rs = make_rsrc((const uint8_t *)p.xs + (int64_t)m0 * (p.k_pad / 32), (uint32_t)(mrows * (p.k_pad / 32)));

    // Activations ride a register ring of DEPTH chunks (slot = (c - c0) %
    // DEPTH) into the double-buffered LDS stage (buffer = (c - c0) & 1).
    u32x4 apre[DEPTH][PIECES];
    uint32_t spre[DEPTH];
    uint32_t abase[PIECES];
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int pc = tid + q * 256, row = pc / (ROWB / 16), kb = (pc % (ROWB / 16)) * 16;
      abase[q] = (uint32_t)row * pitch + (uint32_t)kb;
    }
    const uint32_t xsbase = tid < ROWS ? (uint32_t)(tid * (p.k_pad / 32)) : kOOB;
    auto fetch_a = [&](int aslot, int c) {
#pragma unroll
      for (int q = 0; q < PIECES; ++q) apre[aslot][q] = bload16(rx, c < c1 ? abase[q] + (uint32_t)(c * ROWB) : kOOB);
      if constexpr (!FP8) spre[aslot] = bload4(rs, c < c1 ? xsbase + (uint32_t)(c * 4) : kOOB);
    };
    auto store_a = [&](int aslot, int buf) {
#pragma unroll
      for (int q = 0; q < PIECES; ++q) {
        const int pc = tid + q * 256, row = pc / (ROWB / 16), kb = (pc % (ROWB / 16)) * 16;
        *(u32x4 *)(lds + buf * ABUF + row * STRIDE + kb) = apre[aslot][q];
      }
      if constexpr (!FP8) lds_s[buf][tid] = spre[aslot];
    };

    // Weights: wb[slot][j][q] is the B operand of step j, column tile q (fp4
    // uses its low 4 dwords).  A slot is refilled in place, after the MFMAs
    // that read it, so the ring keeps its registers across the loop.
    // Per-lane bases of this lane's strips, computed once: a load adds the
    // chunk's uniform offset; a strip past the weight keeps kOOB, which
    // stays out of range under any in-weight offset.
    uint32_t bbase[2], sbase[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int strip = s0 + 2 * q + sub;
      const bool live = strip < slim;
      bbase[q] = live ? (uint32_t)strip * (uint32_t)kc * TILE + (uint32_t)((h * 16 + r) * 16) : kOOB;
      sbase[q] = live ? (uint32_t)strip * (uint32_t)kc * 64u + (uint32_t)(r * 4) : kOOB;
    }
    auto bload = [&](int c, int j, int q, int i) -> u32x4 {
      // slot 16(2j + h) + r; its 16-byte half i lives in plane i
      return bload16(rt, c < c1 ? bbase[q] + (uint32_t)(c * TILE + 1024 * i + 512 * j) : kOOB);
    };
    auto sbload = [&](int c, int q) -> uint32_t {  // MXFP4 weight scales of row r, k blocks 0..3
      return bload4(rb, c < c1 ? sbase[q] + (uint32_t)(c * 64) : kOOB);
    };
    i32x8 wb[DEPTH][2][2];
    uint32_t wsb[DEPTH][2];
    // FP8_BLOCK: the wave's 128x128 block scale of chunk c rides the ring with
    // the chunk's weights (one uniform dword load per chunk)
    uint32_t wsv[DEPTH];
    rsrc_t rw = rx;
    if constexpr (FP8) {
      const int sb = s0 < slim ? s0 : slim - 1;
      rw = make_rsrc(w.block_scale + (int64_t)(sb / 8) * w.nbk, (uint32_t)(kc * 4));
    }
    auto wsload = [&](int c) -> uint32_t { return bload4(rw, c < c1 ? (uint32_t)(c * 4) : kOOB); };
    auto refill = [&](int slot, int c, int j, int q) {
      const u32x4 lo = bload(c, j, q, 0);
      wb[slot][j][q][0] = (int)lo[0];
      wb[slot][j][q][1] = (int)lo[1];
      wb[slot][j][q][2] = (int)lo[2];
      wb[slot][j][q][3] = (int)lo[3];
      if constexpr (FP8) {
        const u32x4 hi = bload(c, j, q, 1);
        wb[slot][j][q][4] = (int)hi[0];
        wb[slot][j][q][5] = (int)hi[1];
        wb[slot][j][q][6] = (int)hi[2];
        wb[slot][j][q][7] = (int)hi[3];
      }
    };
    auto fill_slot = [&](int slot, int c) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          wb[slot][j][q] = (i32x8){0, 0, 0, 0, 0, 0, 0, 0};
          refill(slot, c, j, q);
        }
      if constexpr (!FP8)
#pragma unroll
        for (int q = 0; q < 2; ++q) wsb[slot][q] = sbload(c, q);
      if constexpr (FP8) wsv[slot] = wsload(c);
    };
    float mref = 1.0f;

    f32x16 acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][q][e] = 0.0f;

    // Chunk c: barrier; read its activations from its LDS buffer; MFMAs, each
    // weight slot refilled with chunk c+DEPTH after use; then store the
    // activations of chunk c+1 (issued DEPTH chunks earlier) into the other
    // buffer, free since the barrier, and fetch those of chunk c+1+DEPTH.
    // The store's wait for its data thus comes after the chunk's MFMAs are
    // issued.  Loads go out as weights of chunk j-1, then activations of
    // chunk j, in the prologue as in the loop, so every wait is the same.
    __syncthreads();  // the previous segment's reads of buffer 0 are done
    fetch_a(0, c0);
    store_a(0, 0);
#pragma unroll
    for (int j = 1; j <= DEPTH; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      fill_slot(j - 1, c0 + j - 1);
      __builtin_amdgcn_sched_barrier(0);
      fetch_a(j % DEPTH, c0 + j);
    }
    __builtin_amdgcn_sched_barrier(0);

    auto chunk = [&](int slot, int c) {
      const int aslot = (slot + 1) % DEPTH;  // holds the activations of chunk c+1
      const int buf = (c - c0) & 1;
      __syncthreads();  // this chunk's buffer written; the other one no longer read
      const uint8_t *base = lds + buf * ABUF;
      // every activation operand (and MXFP4 scale word) of the chunk, read at once
      i32x8 a[2][MT];
      uint32_t asw[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint8_t *ap = base + row * STRIDE + (FP8 ? 64 * j + 32 * h : 32 * j + 16 * h);
          const u32x4 a0 = *(const u32x4 *)ap;
          if constexpr (FP8) {
            const u32x4 a1 = *(const u32x4 *)(ap + 16);
            a[j][mt] = (i32x8){(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                               (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
          } else {
            a[j][mt] = (i32x8){(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], 0, 0, 0, 0};
          }
        }
        if constexpr (!FP8) asw[mt] = lds_s[buf][row];
      }
      int bsc = 127;
      bool live = true;
      float ratio = 1.0f;  // FP8: applied to each tile just before its first MFMA of the chunk
      if constexpr (FP8) {
        const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(wsv[slot]));
        live = ws != 0.0f;
        if (live) {
          int e;
          const float m = __builtin_frexpf(ws, &e);
          ratio = mref / m;  // exactly 1 when the mantissa repeats
          mref = m;
          bsc = 127 + e;
          bsc = bsc < 0 ? 0 : (bsc > 254 ? 254 : bsc);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        int sbq[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) sbq[q] = FP8 ? bsc : (int)((wsb[slot][q] >> (8 * (2 * j + h))) & 0xff);
        if (live) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int asc = FP8 ? 127 : (int)((asw[mt] >> (8 * (2 * j + h))) & 0xff);
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              if constexpr (FP8)
                if (j == 0) acc[mt][q] *= ratio;
              acc[mt][q] = mfma_scaled32<FP8>(a[j][mt], wb[slot][j][q], acc[mt][q], asc, sbq[q]);
            }
          }
          if constexpr (FP8)
            if (j == 0) {
              // each tile's 16 rescale multiplies run under the previous tile's MFMA
#pragma unroll
              for (int tt = 0; tt < 2 * MT; ++tt) {
                __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // VALU
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
              }
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) refill(slot, c + DEPTH, j, q);
      }
      if constexpr (!FP8)
#pragma unroll
        for (int q = 0; q < 2; ++q) wsb[slot][q] = sbload(c + DEPTH, q);
      if constexpr (FP8) wsv[slot] = wsload(c + DEPTH);
      __builtin_amdgcn_sched_barrier(0);
      store_a(aslot, buf ^ 1);
      fetch_a(aslot, c + 1 + DEPTH);
      __builtin_amdgcn_sched_barrier(0);
    };
    int c = c0;
    for (; c + DEPTH - 1 < c1; c += DEPTH) {
#pragma unroll
      for (int slot = 0; slot < DEPTH; ++slot) chunk(slot, c + slot);
    }
#pragma unroll
    for (int slot = 0; slot + 1 < DEPTH; ++slot)
      if (c + slot < c1) chunk(slot, c + slot);

    // The segment's sum over its chunks, without the per-token factor.
    float sum[ACC];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int e = 0; e < 16; ++e) sum[(mt * 2 + q) * 16 + e] = FP8 ? acc[mt][q][e] * mref : acc[mt][q][e];

    if (t >= 0) {
      // Split tile.  Each piece publishes its partial with agent-scope
      // relaxed atomic stores, waits for them (vmcnt 0), then counts itself
      // in; the last to arrive adds the P partials in piece order -- the
      // same order whichever piece is last, so the result does not depend
      // on timing -- writes the tile and re-arms the counter.
      float *mine = p.part + ((size_t)t * P + piece) * (ACC * 256);
#pragma unroll
      for (int e = 0; e < ACC; ++e)
        __hip_atomic_store(&mine[e * 256 + tid], sum[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();  // every wave's partial stores are complete
      if (tid == 0) lds_last = __hip_atomic_fetch_add(&p.cnt[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == P - 1;
      __syncthreads();
      if (!lds_last) return;
      // All P partials in piece order (this piece's own read back as
      // well), up to 64 values of one piece in flight per round trip: the
      // read-back is a single workgroup's, so its round trips, not its
      // bytes, set its time.
      const rsrc_t rp = make_rsrc(p.part + (size_t)t * P * (ACC * 256), (uint32_t)((size_t)P * ACC * 256 * 4));
      constexpr int HB = ACC < 64 ? ACC : 64;
#pragma unroll
      for (int e = 0; e < ACC; ++e) sum[e] = 0.0f;
      for (int u = 0; u < P; ++u) {
#pragma unroll
        for (int hb = 0; hb < ACC; hb += HB) {
          const uint32_t base_off = (uint32_t)((size_t)u * (ACC * 256) + tid) * 4u;
          float pv[HB];
#pragma unroll
          for (int e = 0; e < HB; ++e)
            pv[e] = __uint_as_float(
                (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rp, (int)(base_off + (hb + e) * 1024u), 0, kSC1));
#pragma unroll
          for (int e = 0; e < HB; ++e) sum[hb + e] += pv[e];
        }
      }
      if (tid == 0) __hip_atomic_store(&p.cnt[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Epilogue: y = sum (x the FP8 per-token scale), rows past M not stored.
    float rowf[MT][16];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) rowf[mt][e] = 1.0f;
    if constexpr (FP8) {
      const rsrc_t rxs = make_rsrc((const float *)p.xs + m0, (uint32_t)mrows * 4u);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          rowf[mt][e] = __builtin_bit_cast(float, bload4(rxs, (uint32_t)(mt * 32 + 8 * (e / 4) + 4 * h + (e % 4)) * 4u));
    }
    if constexpr (SWI) {
      // y[m, j] = silu(gate) * up, one 32x32 tile per exchange
      const int64_t I = w.pair * 16;
      float *xch = (float *)lds;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int64_t j = (int64_t)(j0 + 2 * q) * 16 + (lane & 31);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          float mine[16], up[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) mine[e] = sum[(mt * 2 + q) * 16 + e] * rowf[mt][e];
          swiglu_exchange(xch, wave, lane, mine, up);
          if (wave < 2 && j < I) {
            const int64_t rbase = m0 + mt * 32 + 4 * h;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int64_t row = rbase + 8 * (e / 4) + (e % 4);
              if (row < p.M) store_out(yout, row * out_ld(w) + j, p.y_dtype, silu_mul(mine[e], up[e]));
            }
          }
        }
      }
      return;
    }
    const bool full = m0 + ROWS <= p.M;
    const int64_t ldy = out_ld(w);
  auto body = [&](auto yd, auto chk) __attribute__((always_inline)) {
      typedef decltype(yd) Y;
      constexpr bool CHK = decltype(chk)::value;  // row checks only for the ragged last row tile
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int64_t col = (int64_t)(s0 + 2 * q) * 16 + (lane & 31);
        if (col >= w.N) continue;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int64_t rbase = m0 + mt * 32 + 4 * h;
          typename Y::T *py = (typename Y::T *)yout + rbase * ldy + col;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int rr = 8 * (e / 4) + (e % 4);
            if (!CHK || rbase + rr < p.M) py[rr * ldy] = Y::conv(sum[(mt * 2 + q) * 16 + e] * rowf[mt][e]);
          }
        }
      }
    };
    with_y_dtype(p.y_dtype, [&](auto yd) __attribute__((always_inline)) {
      if (full) body(yd, std::false_type{});
      else body(yd, std::true_type{});
    });
  }
}

// k pieces per tile: 1 (whole tiles) when the tiles fill every resident
// workgroup slot, else as many as fit in one round of slots, each at least
// native_min_chunks chunks long; past one round, a tail split of the last,
// partial round into at most kNativeTailPieces pieces (budget: bytes
// allowed for its partials).  The last piece reads the partials back 64
// values per thread and round trip.
constexpr int kNativeTailPieces = 2;
static SplitPlan native_plan(int fmt, int mt, int occ, int64_t tiles, int64_t kc, size_t budget) {
  SplitPlan s;
  s.tiles = tiles;
  s.tile_part = (size_t)mt * 32 * 256 * sizeof(float);  // MT x 2 column tiles x 16 values per thread
  const int64_t slots = (int64_t)occ * device_cus();
  int64_t P = tiles >= slots ? 1 : slots / tiles;
  const int64_t cap = kc / native_min_chunks(fmt);
  if (P > cap) P = cap;
  s.P = (int)(P < 1 ? 1 : P);
  // partials of at most kGemm32MaxPartBytes, as the 32x32 kernels
  while (s.P > 1 && s.part_bytes() > kGemm32MaxPartBytes) --s.P;
  tail_split(s, slots, kc, budget, kNativeTailPieces);
  return s;
}

// 32-row MFMA tiles per workgroup of a native launch over nt column tiles.
// MXFP4 takes 128-row tiles, or 64-row ones when 128-row tiles would leave
// more than half the CUs without a tile (the 27B k / v at 1024 rows: 32
// tiles, 32 -> 23 us as 64 of 64 rows; at q / o / down, 160-192 tiles,
// 64-row tiles measured 6-18 % slower, and the grouped q / k / v 14 %).
static int native_mt(int fmt, int64_t M, int64_t nt) {
  if (fmt == DIALQ_FORMAT_FP8_BLOCK) return NATIVE_MT_FP8;
  const int64_t rows = 32 * NATIVE_MT_FP4;
  return nt * ((M + rows - 1) / rows) * 2 < device_cus() ? 2 : NATIVE_MT_FP4;
}

template <int FMT, int MT, int OCC, int DEPTH>
static hipError_t native_launch(const WeightView &w, const uint8_t *xq, const void *xs, int64_t M, int64_t k_pad,
                                void *y, int y_dtype, float *part, size_t part_bytes, int *cnt, size_t cnt_count,
                                hipStream_t st, const GemmGroup *grp = nullptr) {
  constexpr int ROWS = 32 * MT;
  constexpr int64_t TILE = FMT == DIALQ_FORMAT_FP8_BLOCK ? 2048 : 1024;
  const int64_t pitch = FMT == DIALQ_FORMAT_FP8_BLOCK ? k_pad : k_pad / 2;
  // 32-bit buffer offsets, with 0x80000000 reserved as the out-of-range offset
  if (w.n_strips * w.k_chunks * TILE >= ((int64_t)1 << 31) || ROWS * pitch >= ((int64_t)1 << 31))
    return hipErrorInvalidValue;
  static_assert(2 * ROWS * ((FMT == DIALQ_FORMAT_FP8_BLOCK ? 128 : 64) + 16) >= 8192,
                "the SwiGLU exchange reuses the staging LDS");
  const int64_t nt = grp ? grp->tbase[grp->nm] : w.pair ? (w.pair + 7) / 8 : (w.n_strips + 15) / 16;
  if (grp)
    for (int j = 0; j < grp->nm; ++j)
      if (grp->wm[j].n_strips * grp->wm[j].k_chunks * TILE >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  const int64_t tiles = nt * ((M + ROWS - 1) / ROWS);
  // the tail budget the workspace was sized with, or the buffer given
  const SplitPlan s = native_plan(FMT, MT, OCC, tiles, w.k_chunks, part_bytes < kTailPartBytes ? part_bytes : kTailPartBytes);
  if (s.grid() > 0x7fffffffLL) return hipErrorInvalidValue;
  if (s.P > 1 && ((size_t)s.nsplit() > cnt_count || s.part_bytes() > part_bytes)) return hipErrorInvalidValue;
  NativeParams p{w, xq, xs, M, k_pad, y, y_dtype, s.P, part, cnt};
  p.W = (int)s.W;
  if (grp) p.g = *grp;
  if (w.pair) k_gemm_native<FMT, MT, OCC, DEPTH, true><<<dim3((unsigned)s.grid()), 256, 0, st>>>(p);
  else k_gemm_native<FMT, MT, OCC, DEPTH, false><<<dim3((unsigned)s.grid()), 256, 0, st>>>(p);
  return hipGetLastError();
}

void native_workspace(int64_t M, const WeightView &w, size_t &part_bytes, size_t &cnt_count, bool tail) {
  const int occ = w.fmt == DIALQ_FORMAT_FP8_BLOCK ? NATIVE_OCC_FP8 : NATIVE_OCC_FP4;
  const int64_t nt = w.pair ? (w.pair + 7) / 8 : (w.n_strips + 15) / 16;
  const int mt = native_mt(w.fmt, M, nt), rows = 32 * mt;
  const int64_t tiles = nt * ((M + rows - 1) / rows);
  const SplitPlan s = native_plan(w.fmt, mt, occ, tiles, w.k_chunks, tail ? kTailPartBytes : 0);
  part_bytes = s.part_bytes();
  cnt_count = (size_t)s.nsplit();
}

// The member table of a grouped native launch (FP8_BLOCK or MXFP4 members of
// one format and K), or false.
static bool native_group_table(const WeightView *ws, void *const *ys, int n, GemmGroup &g) {
  if (n < 2 || n > kGemmMaxGroup) return false;
  if (ws[0].fmt != DIALQ_FORMAT_FP8_BLOCK && ws[0].fmt != DIALQ_FORMAT_MXFP4) return false;
  g.nm = n;
  g.tbase[0] = 0;
  for (int j = 0; j < n; ++j) {
    if (ws[j].fmt != ws[0].fmt || ws[j].K != ws[0].K || ws[j].pair) return false;
    g.wm[j] = ws[j];
    g.ym[j] = ys ? ys[j] : nullptr;
    g.tbase[j + 1] = g.tbase[j] + (int)((ws[j].n_strips + 15) / 16);
  }
  for (int j = n; j < kGemmMaxGroup; ++j) g.tbase[j + 1] = g.tbase[n];
  return true;
}

bool native_group_workspace(int64_t M, const WeightView *ws, int n, size_t &part_bytes, size_t &cnt_count) {
  part_bytes = 0;
  cnt_count = 0;
  GemmGroup g;
  if (M <= 0 || !native_group_table(ws, nullptr, n, g)) return false;
  const bool fp8 = ws[0].fmt == DIALQ_FORMAT_FP8_BLOCK;
  const int occ = fp8 ? NATIVE_OCC_FP8 : NATIVE_OCC_FP4;
  const int mt = native_mt(ws[0].fmt, M, g.tbase[n]), rows = 32 * mt;
  const int64_t tiles = (int64_t)g.tbase[n] * ((M + rows - 1) / rows);
  const SplitPlan s = native_plan(ws[0].fmt, mt, occ, tiles, ws[0].k_chunks, kTailPartBytes);
  part_bytes = s.part_bytes();
  cnt_count = (size_t)s.nsplit();
  return true;
}

hipError_t launch_gemm_native_group(const WeightView *ws, void *const *ys, int n, const uint8_t *xq, const void *xs,
                                    int64_t M, int64_t k_pad, int y_dtype, float *part, size_t part_bytes, int *cnt,
                                    size_t cnt_count, hipStream_t st) {
  GemmGroup g;
  if (!native_group_table(ws, ys, n, g)) return hipErrorNotSupported;
  if (k_pad != ws[0].k_chunks * 128) return hipErrorInvalidValue;
  hipError_t r;
  if (ws[0].fmt == DIALQ_FORMAT_FP8_BLOCK)
    r = native_launch<DIALQ_FORMAT_FP8_BLOCK, NATIVE_MT_FP8, NATIVE_OCC_FP8, NATIVE_DEPTH_FP8>(
        ws[0], xq, xs, M, k_pad, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st, &g);
  else if (native_mt(DIALQ_FORMAT_MXFP4, M, g.tbase[n]) == 2)
    r = native_launch<DIALQ_FORMAT_MXFP4, 2, NATIVE_OCC_FP4, NATIVE_DEPTH_FP4>(
        ws[0], xq, xs, M, k_pad, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st, &g);
  else
    r = native_launch<DIALQ_FORMAT_MXFP4, NATIVE_MT_FP4, NATIVE_OCC_FP4, NATIVE_DEPTH_FP4>(
        ws[0], xq, xs, M, k_pad, ys[0], y_dtype, part, part_bytes, cnt, cnt_count, st, &g);
  if (r == hipSuccess) g_prefill_grouped_launches.fetch_add(1, std::memory_order_relaxed);
  return r;
}

hipError_t launch_gemm_native(const WeightView &w, const uint8_t *xq, const void *xs, int64_t M,
                              int64_t k_pad, void *y, int y_dtype, float *part, size_t part_bytes, int *cnt,
                              size_t cnt_count, hipStream_t st) {
  if (k_pad != w.k_chunks * 128) return hipErrorInvalidValue;
  if (w.fmt == DIALQ_FORMAT_FP8_BLOCK)
    return native_launch<DIALQ_FORMAT_FP8_BLOCK, NATIVE_MT_FP8, NATIVE_OCC_FP8, NATIVE_DEPTH_FP8>(
        w, xq, xs, M, k_pad, y, y_dtype, part, part_bytes, cnt, cnt_count, st);
  if (w.fmt == DIALQ_FORMAT_MXFP4) {
    if (native_mt(w.fmt, M, w.pair ? (w.pair + 7) / 8 : (w.n_strips + 15) / 16) == 2)
      return native_launch<DIALQ_FORMAT_MXFP4, 2, NATIVE_OCC_FP4, NATIVE_DEPTH_FP4>(
          w, xq, xs, M, k_pad, y, y_dtype, part, part_bytes, cnt, cnt_count, st);
    return native_launch<DIALQ_FORMAT_MXFP4, NATIVE_MT_FP4, NATIVE_OCC_FP4, NATIVE_DEPTH_FP4>(
        w, xq, xs, M, k_pad, y, y_dtype, part, part_bytes, cnt, cnt_count, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace dialq

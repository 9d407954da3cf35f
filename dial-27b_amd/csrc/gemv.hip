// Decode GEMV for quantized weights, gfx950: up to 16 rows of x per pass
// (8 for the Q4_K / Q6_K row-packed policies); larger M runs several passes.
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
// Work split: the n_strips * k_chunks tiles, in resident (strip-major)
// order, are cut into ranges of whole strips, one strip per workgroup (the
// kernel also takes equal tile ranges that split strips -- stream-K -- with
// the fix-up below; the launcher uses whole strips, which measured faster).
// The 4 (8 below one strip per CU) waves of a workgroup take interleaved
// tiles of its range; each keeps a register ring of U slots --
// one weight tile, its scales and the activation operands it multiplies, all
// fetched with raw buffer loads whose out-of-range offsets return zeros in
// hardware (no branch, no traffic) -- and refills a slot as soon as it has
// been multiplied, so loads stay in flight and the loop carries no memory
// round trip and no barrier.  When a wave moves on to the next strip it
// parks its accumulator for the finished one in LDS (one slot per strip and
// wave).  After the range is done the waves add the parked slots of each
// strip in wave order; a strip that lies wholly inside the range is written
// out, one shared with neighbouring ranges (at most the first and the last)
// leaves an f32 partial in the workspace, and the last contributor to arrive
// (per-strip counter, reset by that contributor) adds the partials in range
// order -- deterministic.
#include <atomic>

#include "tile_ops.hpp"

namespace dialq {

constexpr int kGemvMaxGroup = 4;  // handles one grouped launch covers

struct GemvParams {
  WeightView w;  // the weight (a grouped launch: its first member)
  const void *x;
  void *y;
  int64_t M;       // total rows of x / y
  int64_t m_base;  // first row handled by this launch
  int y_dtype;
  int G;           // workgroups (tile ranges)
  int spw;         // > 0: range b = strips b*spw .. (b+1)*spw-1 (no strip shared)
  float *ws;       // [G][2][mrows][16] partials of shared strips
  size_t ws_bytes;
  int x_pitch;     // bytes per staged activation row (0: not staged)
  int *cnt;        // [n_strips] arrival counters (zero between launches)
  size_t *query;   // host: non-null = record the workspace bytes, launch nothing
  // Grouped launch (nm > 1, whole strips only): members share x and K;
  // workgroup b takes strip b - sbase[j] of member j, sbase[j] <= b <
  // sbase[j + 1], and writes through ym[j].
  int nm;
  int sbase[kGemvMaxGroup + 1];
  WeightView wm[kGemvMaxGroup];
  void *ym[kGemvMaxGroup];
};

constexpr int kGemvWaves = 4;       // waves per workgroup, whole-strip kernel at >= 1 strip per CU
constexpr int kGemvSmallWaves = 8;  // the same kernel below one strip per CU

// ---------------------------------------------------------------------------
// Activation source.  Small activations (XL) are staged once per workgroup
// into LDS with buffer->LDS DMA, as raw rows of the input dtype at a padded
// row pitch, plus a zero block that lanes whose row is >= mrows read; the
// ring then carries weights only.  Larger ones are fetched per tile into the
// ring (buffer loads, rows >= mrows and k >= K out of range -> zeros).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) uint8_t lds_u8;

typedef __attribute__((address_space(3))) float lds_f32;

// Zero block after the staged rows: lanes that feed zeros read it at the
// same offsets (up to 7 x 64 + 16 bytes) as a staged row of one chunk.
constexpr int kXZeroBytes = 512;

struct Ctx {
  rsrc_t rt, ra, rx;
  const lds_u8 *xl;    // staged rows (XL)
  const lds_u8 *zero;  // kXZeroBytes zero bytes (XL)
  const lds_f32 *xs;   // [mrows][nsub] activation sums per scale sub-block (policies with XS)
  int nsub;            // sub-blocks per row in xs
  int pitch;           // bytes per staged row
  int mrows, K;
};

// Activation sums per scale sub-block of `sub` values, from the staged rows:
// xs[m][b] = sum of x[m][b*sub .. b*sub + sub-1] (the padded tail reads as
// zeros).  Filled by all threads of the workgroup.
template <int ACT>
__device__ __forceinline__ void stage_xsums(const Ctx &cx, lds_f32 *xs, int sub, int threads) {
  constexpr int BY = ActTraits<ACT>::BYTES;
  const int total = cx.mrows * cx.nsub;
  for (int e = threadIdx.x; e < total; e += threads) {
    const int m = e / cx.nsub, b = e - m * cx.nsub;
    const lds_u8 *src = cx.xl + m * cx.pitch + b * sub * BY;
    float a = 0.0f;
    for (int i = 0; i < sub * BY; i += 16) {
      const u32x4 v = *(const u32x4 __attribute__((address_space(3))) *)(src + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (ACT == DIALQ_BF16) a += bf16_bits_to_f32(v[j] & 0xffffu) + bf16_bits_to_f32(v[j] >> 16);
        else if constexpr (ACT == DIALQ_F16 || ACT == kActF16N)
          a += f16_bits_to_f32(v[j] & 0xffffu) + f16_bits_to_f32(v[j] >> 16);
        else a += __uint_as_float(v[j]);
      }
    }
    xs[e] = a;
  }
}

template <int ACT, bool XL>
__device__ __forceinline__ XRaw<ACT> x_fetch(const Ctx &cx, int row, int k, bool valid) {
  constexpr int BY = ActTraits<ACT>::BYTES;
  XRaw<ACT> v;
  if constexpr (XL) {
    const lds_u8 *src = (row < cx.mrows) ? cx.xl + row * cx.pitch + k * BY : cx.zero;
    v.a = *(const u32x4 __attribute__((address_space(3))) *)src;
    if constexpr (ACT == DIALQ_F32) v.b = *(const u32x4 __attribute__((address_space(3))) *)(src + 16);
  } else {
    const uint32_t xo = ((uint32_t)row * (uint32_t)cx.K + (uint32_t)k) * BY;
    v = xraw_load<ACT>(cx.rx, (valid && k < cx.K) ? xo : kOOB);
  }
  return v;
}

// Weight tile and its scales for tile (strip s, chunk c): every load issued
// unconditionally (`valid` = false turns them into out-of-range loads).
template <int FMT>
__device__ __forceinline__ void tile_fill(RawTile &t, const WeightView &w, const Ctx &cx, int s, int c, bool valid,
                                          int lane) {
  typedef FmtTraits<FMT> T;
  const int r = lane & 15, g = lane >> 4;
  const uint32_t tidx = (uint32_t)s * (uint32_t)w.k_chunks + (uint32_t)c;
  t.s0 = 0;
  t.hdr = (u32x4){0, 0, 0, 0};
  if constexpr (FMT == DIALQ_FORMAT_Q6_K) {  // three 1 KB planes, 16 B per lane each
    const uint32_t off = valid ? tidx * 3072 + lane * 16 : kOOB;
    t.a = sload16(cx.rt, off);
    t.b = sload16(cx.rt, valid ? off + 1024 : kOOB);
    t.hdr = sload16(cx.rt, valid ? off + 2048 : kOOB);
    t.sc = sload16(cx.ra, valid ? tidx * 288 + r * 16 : kOOB);
    t.s0 = sload2(cx.ra, valid ? tidx * 288 + 256 + r * 2 : kOOB);
    return;
  }
  const uint32_t off = valid ? tidx * (64 * T::LANE) + lane * 16 : kOOB;  // plane 0
  t.a = sload16(cx.rt, off);
  t.b = (u32x4){0, 0, 0, 0};
  if constexpr (T::LANE == 32) t.b = sload16(cx.rt, valid ? off + 1024 : kOOB);  // plane 1
  if constexpr (FMT == DIALQ_FORMAT_Q8_0) t.s0 = sload4(cx.ra, valid ? tidx * 64 + r * 4 : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_Q4_K) t.hdr = sload16(cx.ra, valid ? tidx * 256 + r * 16 : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_NVFP4) t.s0 = sload2(cx.ra, valid ? tidx * 128 + r * 8 + 2 * g : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_MXFP4) t.s0 = sload1(cx.ra, valid ? tidx * 64 + r * 4 + g : kOOB);
  else if constexpr (FMT == DIALQ_FORMAT_FP8_BLOCK)  // shared by 8 strips: default cache policy
    t.s0 = bload4(cx.ra, valid ? ((uint32_t)((s * 16) / 128) * (uint32_t)w.nbk + (uint32_t)c) * 4 : kOOB);
}

template <int ACT, int N, bool XL>
struct XRing {
  XRaw<ACT> v[N];
};
template <int ACT, int N>
struct XRing<ACT, N, true> {};

// ---------------------------------------------------------------------------
// Per-format ring slot (policy): fill() issues the loads of one tile,
// compute() multiplies a filled slot into the accumulator.
// ---------------------------------------------------------------------------
template <int FMT, int ACT, bool XL>
struct GenericPolicy {
  typedef FmtTraits<FMT> T;
  static constexpr int XACT = ACT;
  static constexpr int XSUB = 0;  // no activation-sum table
  static constexpr int NV = 4;  // accumulator values per lane
  struct Slot {
    RawTile t;
    int c;
    XRing<ACT, T::NX, XL> x;
  };
  struct Acc {
    f32x4 v;
  };
  static __device__ __forceinline__ void zero(Acc &a) { a.v = (f32x4){0.0f, 0.0f, 0.0f, 0.0f}; }
  static __device__ __forceinline__ void fill(Slot &sl, const WeightView &w, const Ctx &cx, int s, int c, bool valid,
                                              int lane) {
    tile_fill<FMT>(sl.t, w, cx, s, c, valid, lane);
    sl.c = c;
    if constexpr (!XL) {
      const int r = lane & 15, g = lane >> 4;
#pragma unroll
      for (int t = 0; t < T::NX; ++t) sl.x.v[t] = x_fetch<ACT, false>(cx, r, c * T::CHUNK + T::xk(t, g), valid);
    }
  }
  static __device__ __forceinline__ void compute(const Slot &sl, Acc &a, const Ctx &cx) {
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    XOp<ACT> xo[T::NX];
#pragma unroll
    for (int t = 0; t < T::NX; ++t) {
      if constexpr (XL) xo[t] = xraw_to_op<ACT>(x_fetch<ACT, true>(cx, r, sl.c * T::CHUNK + T::xk(t, g), true));
      else xo[t] = xraw_to_op<ACT>(sl.x.v[t]);
    }
    bops_mac<FMT, ACT>(make_bops<FMT, ActTraits<ACT>::F16OP>(sl.t), xo, a.v);
  }
  static __device__ __forceinline__ void values(const Acc &a, float (&v)[NV], int (&mrow)[NV], int lane) {
    const int g = lane >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a.v[i];
      mrow[i] = 4 * g + i;
    }
  }
};

// Q4_K, M <= 4*RP: rows of the A operand are (row m' = rho/4, sub-block
// jj = rho%4) pairs, so MFMA t (sub-block t of the super-block) writes
// partial dot products D_t[m'][n] into accumulator rows 4m' + t%4 (the other
// lanes feed zeros), and every lane ends up owning one output (m' = l/16) and
// four sub-blocks (i = 0..3, plus 4..7 in the second accumulator): the
// per-sub-block scales cost 4 FMAs per accumulator instead of 4 per row group
// per sub-block.  Weights enter as bf16(128 + q) (f16(1024 + q) for f16
// activations); the offset and the dmin*m
// term use the per-sub-block activation sums X_t[m'] from a second MFMA with
// a ones operand:  y += s1*D - (128*s1 + dmin*m)*X.  RP passes cover rows
// 4*pass + m'.
template <int ACT, int RP, bool XL, bool XS>
struct Q4kRowsPolicy {
  static constexpr int XACT = ACT;
  static constexpr int NV = RP;
  static constexpr int XSUB = XS ? 32 : 0;  // XS: sums from the staged table, no ones-operand MFMA
  struct Slot {
    RawTile t;
    int c;
    XRing<ACT, 2 * RP, XL> x;  // [q][h]: sub-blocks jj and jj + 4 of row 4q + mq
  };
  struct Acc {
    float v[RP];
  };
  static __device__ __forceinline__ void zero(Acc &a) {
#pragma unroll
    for (int q = 0; q < RP; ++q) a.v[q] = 0.0f;
  }
  static __device__ __forceinline__ int xk(int c, int h, int lane) {
    return c * 256 + 32 * ((lane & 3) + 4 * h) + 8 * (lane >> 4);
  }
  static __device__ __forceinline__ void fill(Slot &sl, const WeightView &w, const Ctx &cx, int s, int c, bool valid,
                                              int lane) {
    tile_fill<DIALQ_FORMAT_Q4_K>(sl.t, w, cx, s, c, valid, lane);
    sl.c = c;
    if constexpr (!XL) {
      const int mq = (lane & 15) >> 2;
#pragma unroll
      for (int q = 0; q < RP; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h) sl.x.v[2 * q + h] = x_fetch<ACT, false>(cx, 4 * q + mq, xk(c, h, lane), valid);
    }
  }
  static constexpr bool F16 = ActTraits<ACT>::F16OP;  // f16(1024 + q) codes, f16 MFMAs
  static constexpr bool ONEPART = ACT == DIALQ_BF16 || F16;
  static __device__ __forceinline__ void compute(const Slot &sl, Acc &acc, const Ctx &cx) {
    const int lane = threadIdx.x & 63, jj = lane & 3, mq = (lane & 15) >> 2;
    constexpr uint32_t ONE = F16 ? 0x3c003c00u : 0x3f803f80u;
    constexpr float OFF = F16 ? 1024.0f : 128.0f;
    const u32x4 ones = {ONE, ONE, ONE, ONE};
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const u32x4 hd = sl.t.hdr;
    const float d = f16_bits_to_f32(hd[0] & 0xffffu), dmin = f16_bits_to_f32(hd[0] >> 16);
    const uint32_t sc_lo = hd[1] & 0x3f3f3f3fu;                                   // sc[0..3]
    const uint32_t m_lo = hd[2] & 0x3f3f3f3fu;                                    // m[0..3]
    const uint32_t sc_hi = (hd[3] & 0x0f0f0f0fu) | ((hd[1] >> 2) & 0x30303030u);  // sc[4..7]
    const uint32_t m_hi = ((hd[3] >> 4) & 0x0f0f0f0fu) | ((hd[2] >> 2) & 0x30303030u);
    const uint32_t qd[8] = {sl.t.a[0], sl.t.a[1], sl.t.a[2], sl.t.a[3], sl.t.b[0], sl.t.b[1], sl.t.b[2], sl.t.b[3]};
#pragma unroll
    for (int q = 0; q < RP; ++q) {
      f32x4 cq[2] = {zero, zero}, cs[2] = {zero, zero};
      if constexpr (XL && ONEPART) {
        // one-part operands straight from the staged rows: a lane outside
        // MFMA t's sub-block (or past the last row) reads the zero block
        const int row = 4 * q + mq;
        const lds_u8 *rowp = cx.xl + row * cx.pitch + (sl.c * 256 + 8 * (lane >> 4)) * 2;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const u32x4 wb = nib8_off<F16>(qd[2 * (t >> 1)], qd[2 * (t >> 1) + 1], (t & 1) ? 4 : 0);
          const lds_u8 *src = ((jj == (t & 3) && row < cx.mrows) ? rowp : cx.zero) + 64 * t;
          XOp<ACT> av;
          av.hi = *(const u32x4 __attribute__((address_space(3))) *)src;
          cq[t >> 2] = mfma_x<ACT>(av, wb, cq[t >> 2]);
          if constexpr (!XS) cs[t >> 2] = mfma_x<ACT>(av, ones, cs[t >> 2]);
        }
      } else {
        XOp<ACT> xa, xb;
        if constexpr (XL) {
          xa = xraw_to_op<ACT>(x_fetch<ACT, true>(cx, 4 * q + mq, xk(sl.c, 0, lane), true));
          xb = xraw_to_op<ACT>(x_fetch<ACT, true>(cx, 4 * q + mq, xk(sl.c, 1, lane), true));
        } else {
          xa = xraw_to_op<ACT>(sl.x.v[2 * q]);
          xb = xraw_to_op<ACT>(sl.x.v[2 * q + 1]);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const u32x4 wb = nib8_off<F16>(qd[2 * (t >> 1)], qd[2 * (t >> 1) + 1], (t & 1) ? 4 : 0);
          const bool on = (jj == (t & 3));
          const XOp<ACT> &src = (t < 4) ? xa : xb;
          XOp<ACT> av;
          av.hi = on ? src.hi : (u32x4){0, 0, 0, 0};
          if constexpr (ActTraits<ACT>::PARTS == 2) av.lo = on ? src.lo : (u32x4){0, 0, 0, 0};
          cq[t >> 2] = mfma_x<ACT>(av, wb, cq[t >> 2]);
          if constexpr (!XS) cs[t >> 2] = mfma_x<ACT>(av, ones, cs[t >> 2]);
        }
      }
      if constexpr (XS) {
        // rows 4g+i of the accumulators: m' = g, sub-blocks i and i + 4
        const int g = lane >> 4, mr = (4 * q + g) < cx.mrows ? 4 * q + g : cx.mrows - 1;
        const lds_f32 *xr = cx.xs + mr * cx.nsub + sl.c * 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cs[0][i] = xr[i];
          cs[1][i] = xr[4 + i];
        }
      }
      // lane (g, r) holds rows 4g+i: m' = g, sub-block i (+4 in [1]);
      // s1*D - (OFF*s1 + dmin*m)*X = d*sc*(D - OFF X) - dmin*m*X
      float sa = 0.0f, sm = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sa = __builtin_fmaf((float)((sc_lo >> (8 * i)) & 0xffu), __builtin_fmaf(-OFF, cs[0][i], cq[0][i]), sa);
        sa = __builtin_fmaf((float)((sc_hi >> (8 * i)) & 0xffu), __builtin_fmaf(-OFF, cs[1][i], cq[1][i]), sa);
        sm = __builtin_fmaf((float)((m_lo >> (8 * i)) & 0xffu), cs[0][i], sm);
        sm = __builtin_fmaf((float)((m_hi >> (8 * i)) & 0xffu), cs[1][i], sm);
      }
      acc.v[q] = __builtin_fmaf(d, sa, __builtin_fmaf(-dmin, sm, acc.v[q]));
    }
  }
  static __device__ __forceinline__ void values(const Acc &a, float (&v)[NV], int (&mrow)[NV], int lane) {
    const int g = lane >> 4;
#pragma unroll
    for (int q = 0; q < RP; ++q) {
      v[q] = a.v[q];
      mrow[q] = 4 * q + g;
    }
  }
};

// Q6_K, M <= 4*RP: the row packing of the Q4_K policy with 16-value
// sub-blocks.  A 32-k slice t spans sub-blocks 2t (lane groups g < 2) and
// 2t + 1 (g >= 2), so A row rho = 4m' + jj feeds sub-block 4u + jj of
// group u = t/2 from the lanes with g/2 == jj%2 in the slices with
// t%2 == jj/2: each lane fetches four activation operands per row pass
// (t = 2u + jj/2), and MFMAs 2u, 2u+1 leave D_{4u+jj}[m'][n] in rows
// 4m' + jj of accumulator u.  Weights enter as bf16(128 + q) (f16(1024 + q)
// for f16 activations, offset 1056 below); with X the
// sub-block's activation sums (ones operand), y += d*sc*(D - 160 X).
template <int ACT, int RP, bool XL, bool XS>
struct Q6kRowsPolicy {
  static constexpr int XACT = ACT;
  static constexpr int NV = RP;
  static constexpr int XSUB = XS ? 16 : 0;  // XS: sums from the staged table, no ones-operand MFMA
  struct Slot {
    RawTile t;
    int c;
    XRing<ACT, 4 * RP, XL> x;  // [q][u]: slice 2u + jj/2 of row 4q + mq
  };
  struct Acc {
    float v[RP];
  };
  static __device__ __forceinline__ void zero(Acc &a) {
#pragma unroll
    for (int q = 0; q < RP; ++q) a.v[q] = 0.0f;
  }
  static __device__ __forceinline__ int xk(int c, int u, int lane) {
    return c * 256 + 32 * (2 * u + ((lane & 3) >> 1)) + 8 * (lane >> 4);
  }
  static __device__ __forceinline__ void fill(Slot &sl, const WeightView &w, const Ctx &cx, int s, int c, bool valid,
                                              int lane) {
    tile_fill<DIALQ_FORMAT_Q6_K>(sl.t, w, cx, s, c, valid, lane);
    sl.c = c;
    if constexpr (!XL) {
      // lanes whose lane group never matches their row's sub-block feed zeros
      const int mq = (lane & 15) >> 2;
      const bool used = valid && ((lane >> 5) & 1) == (lane & 1);
#pragma unroll
      for (int q = 0; q < RP; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) sl.x.v[4 * q + u] = x_fetch<ACT, false>(cx, 4 * q + mq, xk(c, u, lane), used);
    }
  }
  static constexpr bool F16 = ActTraits<ACT>::F16OP;  // f16(1024 + q) codes, f16 MFMAs
  static constexpr bool ONEPART = ACT == DIALQ_BF16 || F16;
  static __device__ __forceinline__ void compute(const Slot &sl, Acc &acc, const Ctx &cx) {
    const int lane = threadIdx.x & 63, jj = lane & 3, mq = (lane & 15) >> 2;
    constexpr uint32_t ONE = F16 ? 0x3c003c00u : 0x3f803f80u;
    constexpr float OFF = F16 ? 1056.0f : 160.0f;  // code offset + 32
    const u32x4 ones = {ONE, ONE, ONE, ONE};
    const u32x4 z4 = {0, 0, 0, 0};
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool gmatch = ((lane >> 5) & 1) == (jj & 1);  // g/2 == jj%2
    const float d = f16_bits_to_f32(sl.t.s0 & 0xffffu);
    u32x4 wb[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) wb[t] = q6x8_off<F16>(t < 4 ? sl.t.a : sl.t.b, sl.t.hdr, t);
#pragma unroll
    for (int q = 0; q < RP; ++q) {
      f32x4 cq[4], cs[4];
      const int row = 4 * q + mq;
      const lds_u8 *rowp = cx.xl + row * cx.pitch + (sl.c * 256 + 8 * (lane >> 4)) * 2;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        XOp<ACT> src;
        if constexpr (XL && ONEPART) (void)src;
        else if constexpr (XL) src = xraw_to_op<ACT>(x_fetch<ACT, true>(cx, 4 * q + mq, xk(sl.c, u, lane), true));
        else src = xraw_to_op<ACT>(sl.x.v[4 * q + u]);
        cq[u] = zero;
        cs[u] = zero;
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          const bool on = gmatch && (v == (jj >> 1));
          XOp<ACT> av;
          if constexpr (XL && ONEPART) {
            // one-part operands straight from the staged rows; lanes that
            // feed zeros (or rows past the last) read the zero block
            const lds_u8 *p = ((on && row < cx.mrows) ? rowp : cx.zero) + 64 * (2 * u + v);
            av.hi = *(const u32x4 __attribute__((address_space(3))) *)p;
          } else {
            av.hi = on ? src.hi : z4;
            if constexpr (ActTraits<ACT>::PARTS == 2) av.lo = on ? src.lo : z4;
          }
          cq[u] = mfma_x<ACT>(av, wb[2 * u + v], cq[u]);
          if constexpr (!XS) cs[u] = mfma_x<ACT>(av, ones, cs[u]);
        }
      }
      if constexpr (XS) {
        // rows 4g+i of accumulator u: m' = g, sub-block 4u + i
        const int g = lane >> 4, mr = (4 * q + g) < cx.mrows ? 4 * q + g : cx.mrows - 1;
        const lds_f32 *xr = cx.xs + mr * cx.nsub + sl.c * 16;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) cs[u][i] = xr[4 * u + i];
      }
      // lane (g, r) holds rows 4g+i: m' = g, sub-block 4u + i = byte i of sc[u]
      float sum = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sum = __builtin_fmaf(sbyte_f32(sl.t.sc[u], i), __builtin_fmaf(-OFF, cs[u][i], cq[u][i]), sum);
      acc.v[q] = __builtin_fmaf(d, sum, acc.v[q]);
    }
  }
  static __device__ __forceinline__ void values(const Acc &a, float (&v)[NV], int (&mrow)[NV], int lane) {
    const int g = lane >> 4;
#pragma unroll
    for (int q = 0; q < RP; ++q) {
      v[q] = a.v[q];
      mrow[q] = 4 * q + g;
    }
  }
};

// ---------------------------------------------------------------------------
// The GEMV kernel.  Dynamic LDS: [staged x: mrows * pitch][32 zero bytes]
// [part[j][wave][m][16]: the accumulator of wave `wave` for the j-th strip
// of the range, rows m < mrows only].
// ---------------------------------------------------------------------------
template <typename Pol, int W>
__device__ __forceinline__ void park(float *part, int j, int wave, int mrows, const typename Pol::Acc &acc) {
  constexpr int NV = Pol::NV;
  const int lane = threadIdx.x & 63, r = lane & 15;
  float v[NV];
  int mrow[NV];
  Pol::values(acc, v, mrow, lane);
  float *dst = part + (size_t)(j * W + wave) * mrows * 16;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (mrow[i] < mrows) dst[mrow[i] * 16 + r] = v[i];
}

// Barrier that orders LDS only (no wait on outstanding global loads).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int FMT, typename Pol, int U, bool XL, int WV>
__global__ __launch_bounds__(64 * WV) void k_gemv(GemvParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int W = WV;
  constexpr int BY = ActTraits<Pol::XACT>::BYTES;
  WeightView w = p.w;
  void *yout = p.y;
  int b = blockIdx.x;
  if (p.nm > 1) {  // grouped launch: this workgroup's member (uniform)
    int j = 0;
#pragma unroll
    for (int i = 1; i < kGemvMaxGroup; ++i) j += (i < p.nm && b >= p.sbase[i]) ? 1 : 0;
    w = p.wm[j];
    yout = p.ym[j];
    b -= p.sbase[j];
  }
  const int64_t ldy = out_ld(w);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kc = (int)w.k_chunks;
  const int64_t total = w.n_strips * w.k_chunks;
  int lo, hi;
  if (p.spw > 0) {
    lo = b * p.spw * kc;
    hi = (int)((int64_t)(b + 1) * p.spw * kc < total ? (int64_t)(b + 1) * p.spw * kc : total);
  } else {
    lo = (int)(((int64_t)b * total) / p.G);
    hi = (int)(((int64_t)(b + 1) * total) / p.G);
  }
  const int s_first = lo / kc;
  const int nseg = (hi > lo) ? (hi - 1) / kc - s_first + 1 : 0;
  // SwiGLU epilogue (w.pair > 0): the tile ranges run over virtual strips,
  // 2j = gate strip j and 2j+1 = up strip pair + j, two per workgroup.
  const int pair = (int)w.pair;
  auto phys = [&](int vs) -> int { return pair ? ((vs & 1) ? pair + (vs >> 1) : (vs >> 1)) : vs; };
  const int mrows = (int)((p.M - p.m_base) < 16 ? (p.M - p.m_base) : 16);
  const int slot_floats = mrows * 16;

  Ctx cx;
  cx.mrows = mrows;
  cx.K = (int)w.K;
  cx.pitch = p.x_pitch;
  cx.xl = (const lds_u8 *)smem;
  cx.zero = (const lds_u8 *)smem + (XL ? mrows * p.x_pitch : 0);
  // LDS: [staged x][32 zero bytes][activation sums (XSUB)][parked accumulators]
  constexpr bool XSUMS = XL && Pol::XSUB > 0;
  cx.nsub = XSUMS ? (int)(w.k_chunks * FmtTraits<FMT>::CHUNK / (XSUMS ? Pol::XSUB : 1)) : 0;
  lds_f32 *xsums = (lds_f32 *)(smem + (XL ? mrows * p.x_pitch + kXZeroBytes : 0));
  cx.xs = xsums;
  float *part = (float *)(smem + (XL ? mrows * p.x_pitch + kXZeroBytes : 0) + (size_t)mrows * cx.nsub * 4);
  cx.rt = make_rsrc(w.tiles, (uint32_t)(total * 64 * FmtTraits<FMT>::LANE));
  cx.ra = cx.rt;
  if constexpr (FMT == DIALQ_FORMAT_Q8_0 || FMT == DIALQ_FORMAT_MXFP4)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 64));
  else if constexpr (FMT == DIALQ_FORMAT_Q4_K)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 256));
  else if constexpr (FMT == DIALQ_FORMAT_Q6_K)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 288));
  else if constexpr (FMT == DIALQ_FORMAT_NVFP4)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 128));
  else if constexpr (FMT == DIALQ_FORMAT_FP8_BLOCK)
    cx.ra = make_rsrc(w.block_scale, (uint32_t)(((w.N + 127) / 128) * w.nbk * 4));
  cx.rx = make_rsrc((const uint8_t *)p.x + p.m_base * w.K * BY, (uint32_t)(mrows * w.K * BY));

  if constexpr (XL) {
    // Stage x: 1 KB per DMA instruction (lane l -> bytes 16l..16l+15 of the
    // block); bytes at or past K*BY read as zeros, which pads every row.
    const int row_bytes = w.K * BY;
    const int blocks = p.x_pitch >> 10;  // 1 KB blocks per row (pitch = blocks KB + 64)
    for (int i = wave; i < mrows * blocks; i += W) {
      const int m = i / blocks, kb = (i - m * blocks) << 10;
      const int col = kb + lane * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(cx.rx, (__attribute__((address_space(3))) void *)(smem + m * p.x_pitch + kb),
                                                16, col < row_bytes ? m * row_bytes + col : (int)kOOB, 0, 0, 0);
    }
    if (threadIdx.x < kXZeroBytes / 16)
      *(u32x4 __attribute__((address_space(3))) *)(smem + mrows * p.x_pitch + 16 * threadIdx.x) = (u32x4){0, 0, 0, 0};
  }
  // each wave clears its own parking slots (a wave may skip a strip)
  for (int j = 0; j < nseg; ++j)
    for (int e = lane; e < slot_floats; e += 64) part[(size_t)(j * W + wave) * slot_floats + e] = 0.0f;
  __builtin_amdgcn_sched_barrier(0);

  // fill cursor: tile t = strip s, chunk c
  int t = lo + wave;
  int s = t / kc, c = t - (t / kc) * kc;
  typename Pol::Slot ring[U];
  int slot_s[U];  // strip of the tile in each slot, -1 = none
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool valid = t < hi;
    Pol::fill(ring[u], w, cx, phys(s), c, valid, lane);
    slot_s[u] = valid ? s : -1;
    t += W;
    c += W;
    while (c >= kc) {
      c -= kc;
      ++s;
    }
  }
  if constexpr (XL) lds_barrier();  // staged x visible to all waves
  if constexpr (XSUMS) {
    stage_xsums<Pol::XACT>(cx, xsums, Pol::XSUB, 64 * W);
    lds_barrier();
  }
  typename Pol::Acc acc;
  Pol::zero(acc);
  int cur = slot_s[0];
  while (slot_s[0] >= 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (slot_s[u] >= 0) {
        if (slot_s[u] != cur) {
          park<Pol, W>(part, cur - s_first, wave, mrows, acc);
          Pol::zero(acc);
          cur = slot_s[u];
        }
        Pol::compute(ring[u], acc, cx);
      }
      const bool valid = t < hi;
      Pol::fill(ring[u], w, cx, phys(s), c, valid, lane);
      slot_s[u] = valid ? s : -1;
      t += W;
      c += W;
      while (c >= kc) {
        c -= kc;
        ++s;
      }
    }
  }
  if (cur >= 0) park<Pol, W>(part, cur - s_first, wave, mrows, acc);
  lds_barrier();

  if (pair) {
    // whole gate / up strip pair j (segments 0 and 1): wave 0 writes
    // silu(gate) * up for rows j*16 .. j*16+15 of the [M, 16*pair] output
    if (wave == 0 && nseg == 2) {
      const int r = lane & 15;
      const int64_t ng = (int64_t)(s_first >> 1) * 16 + r, nu = ng + (int64_t)pair * 16;
      const float sg = epilogue_scale<FMT>(w, ng), su = epilogue_scale<FMT>(w, nu);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = lane + 64 * q, m = e >> 4;
        if (e >= slot_floats) continue;
        float gs = 0.0f, us = 0.0f;
        for (int ww = 0; ww < W; ++ww) {
          gs += part[(size_t)ww * slot_floats + e];
          us += part[(size_t)(W + ww) * slot_floats + e];
        }
        store_out(yout, (p.m_base + m) * ldy + ng, p.y_dtype, silu_mul(gs * sg, us * su));
      }
    }
    return;
  }

  // finish: wave j % W takes strip j of the range
  const int r = lane & 15;
  for (int j = wave; j < nseg; j += W) {
    const int sj = s_first + j;
    const int t0 = sj * kc;
    const int64_t n = (int64_t)sj * 16 + r;
    const float scale = epilogue_scale<FMT>(w, n < w.N ? n : w.N - 1);
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = lane + 64 * q;
      float a = 0.0f;
      if (e < slot_floats)
        for (int ww = 0; ww < W; ++ww) a += part[(size_t)(j * W + ww) * slot_floats + e];
      v[q] = a;
    }
    if (lo <= t0 && t0 + kc <= hi) {  // whole strip
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = lane + 64 * q, m = e >> 4;
        if (e < slot_floats && n < w.N) store_out(yout, (p.m_base + m) * ldy + n, p.y_dtype, v[q] * scale);
      }
      continue;
    }
    // Shared strip.  Partials go to the device-coherent level with
    // agent-scope relaxed atomic stores; waiting for them (vmcnt 0) before
    // the counter increment orders them without the L2 write-back that an
    // agent-scope release fence costs on a multi-XCD part.  The last
    // arriver reads them back with device-coherent (sc1) buffer loads,
    // eight contributors per batch so the round trips overlap.
    const int slot = (j == 0) ? 0 : 1;
    float *mine = p.ws + ((size_t)b * 2 + slot) * slot_floats;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = lane + 64 * q;
      if (e < slot_floats) __hip_atomic_store(&mine[e], v[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    // contributors: ranges owning the strip's first .. last tile
    const int bf = (int)((((int64_t)t0 + 1) * p.G - 1) / total);
    const int bl = (int)((((int64_t)t0 + kc) * p.G - 1) / total);
    int last = 0;
    if (lane == 0) last = (__hip_atomic_fetch_add(&p.cnt[sj], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == bl - bf);
    last = __shfl(last, 0);
    if (!last) continue;
    const rsrc_t rw = make_rsrc(p.ws, (uint32_t)p.ws_bytes);
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b0 = bf; b0 <= bl; b0 += 8) {
      float pv[8][4];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int bb = b0 + i;
        // slot of strip sj in range bb: 1 if bb started in an earlier strip
        const int sl = ((((int64_t)bb * total) / p.G) < t0) ? 1 : 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e = lane + 64 * q;
          const uint32_t off = (bb <= bl && e < slot_floats) ? (uint32_t)((((size_t)bb * 2 + sl) * slot_floats + e) * 4) : kOOB;
          pv[i][q] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, (int)off, 0, kSC1));
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] += pv[i][q];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = lane + 64 * q, m = e >> 4;
      if (e < slot_floats && n < w.N) store_out(yout, (p.m_base + m) * ldy + n, p.y_dtype, a[q] * scale);
    }
    if (lane == 0) __hip_atomic_store(&p.cnt[sj], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Dynamic GEMV kernel.  Work is cut into units -- piece p of strip s, the
// chunks [p*cpp, min((p+1)*cpp, kc)) with cpp <= W*U, i.e. at most one ring
// cycle per wave -- handed out at run time, so faster CUs take more units and
// every CU finishes together.  A workgroup has W compute waves and one
// control wave.  The compute waves stream their units' tiles through the
// ring and, after each unit, park their accumulators in LDS and bump the
// unit's LDS counter; they wait on nothing but their own loads and the LDS
// unit queue.  The control wave keeps the queue kDynQueue units ahead (the
// first kDynQueue units of workgroup b are b + j*G, later ones come from a
// global atomic counter) and closes finished units: it adds the W parked
// accumulators in wave order and writes the strip (one piece per strip) or
// publishes the piece's partial; the last piece of a strip to be published
// adds all pieces in piece order and writes the strip -- deterministic.  All
// waits are bounded (kSpinLimit polls without progress by default), so no
// wave can hang; a wait that gives up marks the handle (DynParams::err).
//
// LDS: [ctl: q[kDynQueue], ng, done[kDynQueue]][staged x][32 zero bytes]
//      [park[kDynQueue][W][mrows][16] floats]
// ---------------------------------------------------------------------------
constexpr int kDynWaves = 4;   // compute waves per workgroup (plus one control wave)
constexpr int kDynQueue = 8;   // units queued ahead per workgroup
constexpr int kDynCtlBytes = 128;
constexpr int kSpinLimit = 1 << 22;

struct DynParams {
  WeightView w;
  const void *x;
  void *y;
  int64_t M;       // total rows of x / y
  int64_t m_base;  // first row handled by this launch
  int y_dtype;
  int P;           // pieces per strip
  int cpp;         // chunks per piece
  int NU;          // units: n_strips * P
  int G;           // workgroups
  int x_pitch;     // bytes per staged activation row (0: not staged)
  float *ws;       // [n_strips][P][mrows][16] piece partials (P > 1)
  size_t ws_bytes;
  int *cnt;        // [n_strips] piece counters, then queue head and exit count
  int *err;        // host-visible word set to 1 when a bounded wait gives up
  int spin_limit;  // polls without progress before a wait gives up
  size_t *query;   // host: non-null = record the workspace bytes, launch nothing
  const GemvParams *group;  // host: grouped launch (members, strip bases, outputs), or null
};

// A wave whose bounded wait gave up: the launch's output is incomplete.  The
// word lives in host memory so that the next forward on the handle can see
// it without synchronising.
__device__ __forceinline__ void report_gave_up(const DynParams &p) {
  if ((threadIdx.x & 63) == 0) __hip_atomic_store(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ int lds_load(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(int *p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local"); }
__device__ __forceinline__ void lds_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local"); }

// Unit u -> strip, chunk range.
__device__ __forceinline__ void unit_range(const DynParams &p, int u, int &s, int &c0, int &c1) {
  s = u / p.P;
  c0 = (u - s * p.P) * p.cpp;
  const int e = c0 + p.cpp, kc = (int)p.w.k_chunks;
  c1 = e < kc ? e : kc;
}

// Control wave: add the W parked accumulators of park slot k (wave order).
__device__ __forceinline__ void reduce_park(const float *park_k, int slot_floats, float (&v)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = lane + 64 * q;
    float a = 0.0f;
    if (e < slot_floats)
      for (int ww = 0; ww < kDynWaves; ++ww) a += park_k[ww * slot_floats + e];
    v[q] = a;
  }
}

// Control wave: write rows m < mrows of strip s (16 outputs per row).
template <int FMT>
__device__ __forceinline__ void store_strip(const DynParams &p, int s, int slot_floats, const float (&v)[4]) {
  const WeightView &w = p.w;
  const int lane = threadIdx.x & 63, r = lane & 15;
  const int64_t n = (int64_t)s * 16 + r;
  const float scale = epilogue_scale<FMT>(w, n < w.N ? n : w.N - 1);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = lane + 64 * q, m = e >> 4;
    if (e < slot_floats && n < w.N) store_out(p.y, (p.m_base + m) * out_ld(w) + n, p.y_dtype, v[q] * scale);
  }
}

// Control wave: all P pieces of strip s are published -- add them in piece
// order (device-coherent loads, eight pieces per batch), write the strip and
// rearm its counter.
template <int FMT>
__device__ void finish_strip(const DynParams &p, int s, int slot_floats) {
  const int lane = threadIdx.x & 63;
  const rsrc_t rw = make_rsrc(p.ws + (size_t)s * p.P * slot_floats, (uint32_t)((size_t)p.P * slot_floats * 4));
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int b0 = 0; b0 < p.P; b0 += 8) {
    float pv[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = lane + 64 * q;
        const uint32_t off = (b0 + i < p.P && e < slot_floats) ? (uint32_t)(((b0 + i) * slot_floats + e) * 4) : kOOB;
        pv[i][q] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, (int)off, 0, kSC1));
      }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) a[q] += pv[i][q];
  }
  store_strip<FMT>(p, s, slot_floats, a);
  if (lane == 0) __hip_atomic_store(&p.cnt[s], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Control wave main loop.  Each round: close every unit all compute waves
// have finished (in queue order): one piece per strip -> write the strip;
// otherwise publish the piece's partial with agent-scope stores.  Then, in
// one memory round trip after the stores have completed, count the
// published pieces in (one lane per piece) and grab as many units as there
// are free queue slots; the last piece of a strip to be counted adds up the
// strip.
template <int FMT>
__device__ void control_wave(const DynParams &p, int *q, int *ng, int *done, const float *park, int mrows) {
  constexpr int W = kDynWaves, QD = kDynQueue;
  const int lane = threadIdx.x & 63;
  const int slot_floats = mrows * 16;
  int *head = p.cnt + p.w.n_strips, *exits = head + 1;
  int nq = QD, nclosed = 0, spin = 0;
  bool exhausted = false, end = false;
  for (int j = 0; j < QD; ++j) exhausted = exhausted || (lds_load(&q[j]) < 0);
  int pend = -1, npend = 0;  // lane i < npend holds the strip of published piece i
  while (true) {
    bool prog = false;
    while (!end && nclosed < nq) {
      const int k = nclosed % QD;
      const int u = lds_load(&q[k]);
      if (u < 0) {
        end = true;
        break;
      }
      if (lds_load(&done[k]) != W) break;
      lds_acquire();
      float v[4];
      reduce_park(park + (size_t)k * W * slot_floats, slot_floats, v);
      const int s = u / p.P;
      if (p.P == 1) {
        store_strip<FMT>(p, s, slot_floats, v);
      } else {
        float *mine = p.ws + ((size_t)u) * slot_floats;  // u = s * P + piece
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int e = lane + 64 * qq;
          if (e < slot_floats) __hip_atomic_store(&mine[e], v[qq], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        pend = (lane == npend) ? s : pend;
        ++npend;
      }
      lds_store(&done[k], 0);
      ++nclosed;
      prog = true;
    }
    const int want = exhausted ? 0 : nclosed + QD - nq;
    if (npend > 0 || want > 0) {
      __builtin_amdgcn_s_waitcnt(0);  // published partials have landed
      int old = 0;
      if (lane < npend) old = __hip_atomic_fetch_add(&p.cnt[pend], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane == 63 && want > 0) old = __hip_atomic_fetch_add(head, want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (want > 0) {
        const int h = __builtin_amdgcn_readlane(old, 63) + QD * p.G;
        for (int j = 0; j < want; ++j) {
          int u = h + j;
          if (u >= p.NU) {
            u = -1;
            exhausted = true;
          }
          lds_store(&q[nq % QD], u);
          ++nq;
          if (u < 0) break;
        }
        lds_release();
        lds_store(ng, nq);
      }
      for (int i = 0; i < npend; ++i)
        if (__builtin_amdgcn_readlane(old, i) == p.P - 1) finish_strip<FMT>(p, __builtin_amdgcn_readlane(pend, i), slot_floats);
      npend = 0;
      pend = -1;
      prog = true;
    }
    if (end && npend == 0) break;
    if (prog) {
      spin = 0;
    } else {
      __builtin_amdgcn_s_sleep(1);
      if (++spin > p.spin_limit) {
        report_gave_up(p);
        break;
      }
    }
  }
  // The last workgroup out resets the queue for the next launch.
  if (lane == 0 && __hip_atomic_fetch_add(exits, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.G - 1) {
    __hip_atomic_store(head, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(exits, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int FMT, typename Pol, int U, bool XL>
__global__ __launch_bounds__(64 * (kDynWaves + 1)) void k_gemv_dyn(DynParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int W = kDynWaves, QD = kDynQueue;
  constexpr int BY = ActTraits<Pol::XACT>::BYTES;
  const WeightView &w = p.w;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x;
  const int mrows = (int)((p.M - p.m_base) < 16 ? (p.M - p.m_base) : 16);
  const int slot_floats = mrows * 16;
  int *q = (int *)smem;       // [QD] unit of each queued ordinal (-1: no more)
  int *ng = q + QD;           // ordinals queued so far
  int *done = q + QD + 1;     // [QD] waves finished with the unit in each slot
  uint8_t *xbase = smem + kDynCtlBytes;
  float *park = (float *)(xbase + (XL ? mrows * p.x_pitch + kXZeroBytes : 0));

  Ctx cx;
  cx.mrows = mrows;
  cx.K = (int)w.K;
  cx.pitch = p.x_pitch;
  cx.xl = (const lds_u8 *)xbase;
  cx.zero = (const lds_u8 *)xbase + (XL ? mrows * p.x_pitch : 0);
  cx.xs = nullptr;  // the dynamic kernel's policies take their sums from MFMAs
  cx.nsub = 0;
  const int64_t total = w.n_strips * w.k_chunks;
  cx.rt = make_rsrc(w.tiles, (uint32_t)(total * 64 * FmtTraits<FMT>::LANE));
  cx.ra = cx.rt;
  if constexpr (FMT == DIALQ_FORMAT_Q8_0 || FMT == DIALQ_FORMAT_MXFP4)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 64));
  else if constexpr (FMT == DIALQ_FORMAT_Q4_K)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 256));
  else if constexpr (FMT == DIALQ_FORMAT_Q6_K)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 288));
  else if constexpr (FMT == DIALQ_FORMAT_NVFP4)
    cx.ra = make_rsrc(w.aux, (uint32_t)(total * 128));
  else if constexpr (FMT == DIALQ_FORMAT_FP8_BLOCK)
    cx.ra = make_rsrc(w.block_scale, (uint32_t)(((w.N + 127) / 128) * w.nbk * 4));
  cx.rx = make_rsrc((const uint8_t *)p.x + p.m_base * w.K * BY, (uint32_t)(mrows * w.K * BY));

  // Queue the statically assigned first units; clear the counters.
  if (threadIdx.x < QD) {
    const int u = b + (int)threadIdx.x * p.G;
    lds_store(&q[threadIdx.x], u < p.NU ? u : -1);
    lds_store(&done[threadIdx.x], 0);
  }
  if (threadIdx.x == 0) lds_store(ng, QD);
  if constexpr (XL) {
    if (wave < W) {
      // Stage x: 1 KB per DMA instruction (lane l -> bytes 16l..16l+15 of the
      // block); bytes at or past K*BY read as zeros, which pads every row.
      const int row_bytes = w.K * BY;
      const int blocks = p.x_pitch >> 10;
      for (int i = wave; i < mrows * blocks; i += W) {
        const int m = i / blocks, kb = (i - m * blocks) << 10;
        const int col = kb + lane * 16;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(cx.rx, (__attribute__((address_space(3))) void *)(xbase + m * p.x_pitch + kb),
                                                  16, col < row_bytes ? m * row_bytes + col : (int)kOOB, 0, 0, 0);
      }
    }
    if (threadIdx.x < kXZeroBytes / 16)
      *(u32x4 __attribute__((address_space(3))) *)(xbase + mrows * p.x_pitch + 16 * threadIdx.x) = (u32x4){0, 0, 0, 0};
  }
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();  // queue and counters initialised

  if (wave == W) {
    lds_barrier();  // pairs with the compute waves' second barrier
    control_wave<FMT>(p, q, ng, done, park, mrows);
    return;
  }

  // ---- compute waves ---------------------------------------------------
  typename Pol::Slot ring[U];
  bool valid[U];
  int cur = lds_load(&q[0]);
  {
    int s = 0, c0 = 0, c1 = 0;
    if (cur >= 0) unit_range(p, cur, s, c0, c1);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + wave + W * u;
      valid[u] = cur >= 0 && c < c1;
      Pol::fill(ring[u], w, cx, s, valid[u] ? c : 0, valid[u], lane);
    }
  }
  lds_barrier();  // staged x visible (waits for this wave's DMA, not its ring)
  typename Pol::Acc acc;
  Pol::zero(acc);
  int ord = 0;
  while (cur >= 0) {
    // next unit: wait until the control wave has queued ordinal ord + 1
    int spin = 0;
    while (lds_load(ng) <= ord + 1) {
      if (++spin > p.spin_limit) break;
      __builtin_amdgcn_s_sleep(1);
    }
    lds_acquire();
    const bool gave_up = spin > p.spin_limit;
    if (gave_up) report_gave_up(p);
    const int nxt = gave_up ? -1 : lds_load(&q[(ord + 1) % QD]);
    int s = 0, c0 = 0, c1 = 0;
    if (nxt >= 0) unit_range(p, nxt, s, c0, c1);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (valid[u]) Pol::compute(ring[u], acc, cx);
      const int c = c0 + wave + W * u;
      valid[u] = nxt >= 0 && c < c1;
      Pol::fill(ring[u], w, cx, s, valid[u] ? c : 0, valid[u], lane);
    }
    // park this wave's share of unit `cur` and count it in
    {
      constexpr int NV = Pol::NV;
      const int r = lane & 15;
      float v[NV];
      int mrow[NV];
      Pol::values(acc, v, mrow, lane);
      float *dst = park + ((size_t)(ord % QD) * W + wave) * slot_floats;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (mrow[i] < mrows) dst[mrow[i] * 16 + r] = v[i];
      lds_release();
      if (lane == 0) __hip_atomic_fetch_add(&done[ord % QD], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    Pol::zero(acc);
    cur = nxt;
    ++ord;
  }
}

// ---------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------
int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

// Ring depth: ~96 VGPRs of in-flight weights, scales and activations.
constexpr int ring_depth(int slot_vgprs) {
  return (96 / slot_vgprs) >= 8 ? 8
       : ((96 / slot_vgprs) >= 6 ? 6 : ((96 / slot_vgprs) >= 4 ? 4 : ((96 / slot_vgprs) >= 3 ? 3 : 2)));
}

constexpr int kGemvWgPerCu = 2;          // target ranges per CU
constexpr int kRangeRing = 4;            // ring depth cap of the whole-strip kernel
constexpr int kGemvParkBytes = 16384;    // parking LDS per workgroup
constexpr int kGemvStageBytes = 65536;   // staged-activation LDS per workgroup
constexpr int kGemvSmallStageBytes = 131072;  // the same below one strip per CU (about one workgroup per CU)

// Ranges for one pass of mrows rows: kGemvWgPerCu per CU, more when a range
// would span more strips than its parking LDS holds, never more than tiles.
static int gemv_grid(const WeightView &w, int64_t mrows) {
  const int64_t total = w.n_strips * w.k_chunks;
  const int64_t seg_cap = kGemvParkBytes / (kGemvWaves * mrows * 16 * 4);  // strips per range
  int64_t g = (int64_t)kGemvWgPerCu * device_cus();
  // a range of ceil(total/g) tiles spans at most ceil(total/g)/kc + 2 strips
  const int64_t need = (w.n_strips + seg_cap - 3) / (seg_cap - 2);
  if (g < need) g = need;
  if (g > total) g = total;
  return (int)(g < 1 ? 1 : g);
}

// Bytes per staged activation row: whole 1 KB DMA blocks covering the padded
// k range, plus 64 bytes so that rows start in different LDS banks.
static int stage_pitch(const WeightView &w, int by, int chunk) {
  const int64_t kpad_bytes = w.k_chunks * chunk * by;
  return (int)(((kpad_bytes + 1023) / 1024) * 1024 + 64);
}

// Strips per workgroup.  One (no strip is shared, so no cross-workgroup
// fix-up): measured on the 27B gate shape, one strip per workgroup and four
// loads in flight per wave stream 17% faster than two strips and eight loads
// -- several resident workgroups per CU, each with a shallow ring, keep more
// of HBM busy than a few deep ones (a plain read kernel shows the same).
// 0 selects equal tile ranges (stream-K), used when several activation rows
// ride the ring with the weights (too large to stage): there each tile's
// activation fetch lengthens the loop, and balancing the tiles over 2
// workgroups per CU measured 17-23 % faster on the 27B down shape at M = 4-8
// (10-18 % for Q4_K); with staged activations it is slower.
static int gemv_spw(const WeightView &w, int64_t mrows, bool staged) {
  (void)w;
  return (!staged && mrows > 1) ? 0 : 1;
}

template <int FMT, typename Pol, int U, bool XL, int WV>
static hipError_t launch_ranges(GemvParams &p, hipStream_t st) {
  const int64_t mrows = (p.M - p.m_base) < 16 ? (p.M - p.m_base) : 16;
  const int64_t total = p.w.n_strips * p.w.k_chunks;
  p.spw = p.w.pair ? 2 : gemv_spw(p.w, mrows, XL);  // SwiGLU: whole gate / up strip pairs
  p.G = p.spw > 0 ? (int)((p.w.n_strips + p.spw - 1) / p.spw) : gemv_grid(p.w, mrows);
  if (p.nm > 1) p.G = p.sbase[p.nm];  // grouped: one workgroup per strip of every member
  const int64_t per = p.spw > 0 ? p.spw * p.w.k_chunks : (total + p.G - 1) / p.G;
  const int64_t nseg = p.spw > 0 ? p.spw : per / p.w.k_chunks + 2;
  const size_t park = (size_t)nseg * WV * mrows * 16 * sizeof(float);
  if (park > (size_t)kGemvParkBytes) return hipErrorInvalidConfiguration;
  const size_t need = p.spw == 0 ? (size_t)p.G * 2 * mrows * 16 * sizeof(float) : 0;
  if (p.query) {
    if (need > *p.query) *p.query = need;
    return hipSuccess;
  }
  if (need > p.ws_bytes) return hipErrorInvalidValue;
  const size_t xsums = (XL && Pol::XSUB > 0)
                           ? (size_t)mrows * (p.w.k_chunks * FmtTraits<FMT>::CHUNK / (Pol::XSUB > 0 ? Pol::XSUB : 1)) * 4
                           : 0;
  const size_t lds = park + (XL ? (size_t)mrows * p.x_pitch + kXZeroBytes : 0) + xsums;
  k_gemv<FMT, Pol, U, XL, WV><<<(unsigned)p.G, 64 * WV, lds, st>>>(p);
  return hipGetLastError();
}

template <int FMT, typename Pol, int U, bool XL>
static hipError_t launch_dyn(DynParams &p, int64_t mrows, hipStream_t st) {
  const int kc = (int)p.w.k_chunks;
  p.P = (kc + kDynWaves * U - 1) / (kDynWaves * U);
  p.cpp = (kc + p.P - 1) / p.P;
  p.NU = (int)(p.w.n_strips * p.P);
  p.G = kGemvWgPerCu * device_cus();
  if (p.G > p.NU) p.G = p.NU;
  const size_t need = p.P > 1 ? (size_t)p.w.n_strips * p.P * mrows * 16 * sizeof(float) : 0;
  if (p.query) {
    if (need > *p.query) *p.query = need;
    return hipSuccess;
  }
  if (need > p.ws_bytes) return hipErrorInvalidValue;
  const size_t lds = kDynCtlBytes + (XL ? (size_t)mrows * p.x_pitch + kXZeroBytes : 0) +
                     (size_t)kDynQueue * kDynWaves * mrows * 16 * sizeof(float);
  k_gemv_dyn<FMT, Pol, U, XL><<<(unsigned)p.G, 64 * (kDynWaves + 1), lds, st>>>(p);
  return hipGetLastError();
}

// Whole-strip ranges (no strip shared between workgroups) whenever the
// activations can be staged: 4 waves per workgroup at one strip per CU or
// more, 8 below.  The dynamic kernel, whose small units keep every CU busy,
// takes the matrices with fewer strips than CUs whose activations are too
// large to stage.
template <int FMT, int ACT, template <int, int, bool, bool> class PolT, int A, int U_XL, int U_X>
static hipError_t launch_pol(DynParams &d, int64_t mrows, hipStream_t st) {
  constexpr int BY = ActTraits<ACT>::BYTES;
  const bool xl = mrows * stage_pitch(d.w, BY, FmtTraits<FMT>::CHUNK) + kXZeroBytes <= kGemvStageBytes;
  constexpr int UR = U_XL < kRangeRing ? U_XL : kRangeRing;
  if (d.group) {
    // Grouped launch: the strips of every member, whole strips with staged
    // activations only (4 waves per workgroup at one strip per CU or more,
    // 8 below); other configurations run one launch per member.
    const int pitch = stage_pitch(d.w, BY, FmtTraits<FMT>::CHUNK);
    const int total = d.group->sbase[d.group->nm];
    if (d.w.pair || mrows * pitch + kXZeroBytes > (total >= device_cus() ? kGemvStageBytes : kGemvSmallStageBytes))
      return hipErrorNotSupported;
    GemvParams p = *d.group;
    p.x = d.x;
    p.M = d.M;
    p.m_base = d.m_base;
    p.y_dtype = d.y_dtype;
    p.x_pitch = pitch;
    p.query = d.query;
    if (total >= device_cus()) return launch_ranges<FMT, PolT<A, ACT, true, true>, UR, true, kGemvWaves>(p, st);
    return launch_ranges<FMT, PolT<A, ACT, true, true>, UR, true, kGemvSmallWaves>(p, st);
  }
  if (d.w.pair) {
    // SwiGLU epilogue: one gate / up strip pair per workgroup, never split
    // (the pair's two sums meet in the workgroup's parking LDS)
    // 8 waves: each of the pair's strips streams as a 4-wave plain workgroup
    // would, so the rounds of workgroups over the CUs match the plain launch
    GemvParams p{d.w, d.x, d.y, d.M, d.m_base, d.y_dtype, 1, 0, d.ws, d.ws_bytes, 0, d.cnt, d.query};
    const int pitch = stage_pitch(d.w, BY, FmtTraits<FMT>::CHUNK);
    if (mrows * pitch + kXZeroBytes <= kGemvSmallStageBytes) {
      p.x_pitch = pitch;
      return launch_ranges<FMT, PolT<A, ACT, true, true>, UR, true, kGemvSmallWaves>(p, st);
    }
    return launch_ranges<FMT, PolT<A, ACT, false, false>, (U_X < kRangeRing ? U_X : kRangeRing), false, kGemvWaves>(
        p, st);
  }
  if (d.w.n_strips >= device_cus()) {
    GemvParams p{d.w, d.x, d.y, d.M, d.m_base, d.y_dtype, 1, 0, d.ws, d.ws_bytes, 0, d.cnt, d.query};
    p.x_pitch = xl ? stage_pitch(d.w, BY, FmtTraits<FMT>::CHUNK) : 0;
    if (xl) return launch_ranges<FMT, PolT<A, ACT, true, true>, UR, true, kGemvWaves>(p, st);
    return launch_ranges<FMT, PolT<A, ACT, false, false>, (U_X < kRangeRing ? U_X : kRangeRing), false, kGemvWaves>(
        p, st);
  }
  if (mrows * stage_pitch(d.w, BY, FmtTraits<FMT>::CHUNK) + kXZeroBytes <= kGemvSmallStageBytes) {
    // Fewer strips than CUs, activations staged: one strip per workgroup of
    // kGemvSmallWaves waves, so each wave streams a short run of tiles and
    // nothing is reduced across workgroups.  Measured at M = 1..4 with
    // K = 5120: 5.3 us for 256..2048 rows where the work queue took 6.8-9.4
    // (3072 rows: 5.7 against 12.0); K = 17408 at 1024-2048 rows 25-35 %
    // faster.
    GemvParams p{d.w, d.x, d.y, d.M, d.m_base, d.y_dtype, 1, 0, d.ws, d.ws_bytes, 0, d.cnt, d.query};
    p.x_pitch = stage_pitch(d.w, BY, FmtTraits<FMT>::CHUNK);
    return launch_ranges<FMT, PolT<A, ACT, true, true>, UR, true, kGemvSmallWaves>(p, st);
  }
  d.x_pitch = 0;
  return launch_dyn<FMT, PolT<A, ACT, false, false>, U_X, false>(d, mrows, st);
}

// Adapters so both policies take <first, ACT, XL> template arguments.
template <int FMT, int ACT, bool XL, bool XS>
using GenericPol = GenericPolicy<FMT, ACT, XL>;
template <int RP, int ACT, bool XL, bool XS>
using Q4kRowsPol = Q4kRowsPolicy<ACT, RP, XL, XS>;
template <int RP, int ACT, bool XL, bool XS>
using Q6kRowsPol = Q6kRowsPolicy<ACT, RP, XL, XS>;

template <int FMT, int ACT>
static hipError_t gemv_dispatch(const WeightView &w, const void *x, int64_t M, void *y, int y_dtype,
                                float *ws, size_t ws_bytes, int *cnt, int *err, size_t *query, hipStream_t st,
                                const GemvParams *group = nullptr) {
  typedef FmtTraits<FMT> T;
  constexpr int XV = (ACT == DIALQ_F32) ? 8 : 4;  // VGPRs per 8-element activation operand
  constexpr bool KQ = FMT == DIALQ_FORMAT_Q4_K || FMT == DIALQ_FORMAT_Q6_K;
  constexpr int TV = T::LANE / 4 + (FMT == DIALQ_FORMAT_Q4_K ? 4 : FMT == DIALQ_FORMAT_Q6_K ? 5 : 1) + 1;  // tile + scales + chunk
  const int rows_per_pass = (KQ && M <= 8) ? 8 : 16;
  for (int64_t mb = 0; mb < M; mb += rows_per_pass) {
    const int64_t rem = M - mb, mrows = rem < 16 ? rem : 16;
    DynParams p{w, x, y, M, mb, y_dtype, 1, 1, 1, 1, 0, ws, ws_bytes, cnt, err, gemv_wait_limit(), query, group};
    hipError_t e;
    if constexpr (FMT == DIALQ_FORMAT_Q4_K) {
      if (rem <= 4)
        e = launch_pol<FMT, ACT, Q4kRowsPol, 1, ring_depth(TV), ring_depth(TV + 2 * XV)>(p, mrows, st);
      else if (rem <= 8)
        e = launch_pol<FMT, ACT, Q4kRowsPol, 2, ring_depth(TV), ring_depth(TV + 4 * XV)>(p, mrows, st);
      else
        e = launch_pol<FMT, ACT, GenericPol, FMT, ring_depth(TV), ring_depth(TV + T::NX * XV)>(p, mrows, st);
    } else if constexpr (FMT == DIALQ_FORMAT_Q6_K) {
      if (rem <= 4)
        e = launch_pol<FMT, ACT, Q6kRowsPol, 1, ring_depth(TV), ring_depth(TV + 4 * XV)>(p, mrows, st);
      else if (rem <= 8)
        e = launch_pol<FMT, ACT, Q6kRowsPol, 2, ring_depth(TV), ring_depth(TV + 8 * XV)>(p, mrows, st);
      else
        e = launch_pol<FMT, ACT, GenericPol, FMT, ring_depth(TV), ring_depth(TV + T::NX * XV)>(p, mrows, st);
    } else {
      e = launch_pol<FMT, ACT, GenericPol, FMT, ring_depth(TV), ring_depth(TV + T::NX * XV)>(p, mrows, st);
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}


template <int FMT>
static hipError_t gemv_act(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y,
                           int y_dtype, float *ws, size_t ws_bytes, int *cnt, int *err, size_t *query,
                           hipStream_t st, const GemvParams *group) {
  switch (x_dtype) {
    case DIALQ_BF16: return gemv_dispatch<FMT, DIALQ_BF16>(w, x, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    // f16 activations feed f16 MFMAs as they are (f16 weight operands);
    // MXFP4's scaled codes need bf16's exponent range (hi / lo parts)
    case DIALQ_F16:
      return gemv_dispatch<FMT, FMT == DIALQ_FORMAT_MXFP4 ? DIALQ_F16 : kActF16N>(w, x, M, y, y_dtype, ws, ws_bytes,
                                                                                 cnt, err, query, st, group);
    case DIALQ_F32: return gemv_dispatch<FMT, DIALQ_F32>(w, x, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
  }
  return hipErrorInvalidValue;
}

namespace {
std::atomic<int> g_wait_limit{kSpinLimit};
}

int gemv_wait_limit() { return g_wait_limit.load(std::memory_order_relaxed); }

void set_gemv_wait_limit(int64_t polls) {
  g_wait_limit.store(polls < 0 ? kSpinLimit : (int)(polls < kSpinLimit ? polls : kSpinLimit), std::memory_order_relaxed);
}

static hipError_t gemv_fmt(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y, int y_dtype,
                           float *ws, size_t ws_bytes, int *cnt, int *err, size_t *query, hipStream_t st,
                           const GemvParams *group = nullptr) {
  switch (w.fmt) {
    case DIALQ_FORMAT_W8A16: return gemv_act<DIALQ_FORMAT_W8A16>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    case DIALQ_FORMAT_FP8_ROW: return gemv_act<DIALQ_FORMAT_FP8_ROW>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    case DIALQ_FORMAT_Q8_0: return gemv_act<DIALQ_FORMAT_Q8_0>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    case DIALQ_FORMAT_FP8_BLOCK:
      return gemv_act<DIALQ_FORMAT_FP8_BLOCK>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    case DIALQ_FORMAT_NVFP4: return gemv_act<DIALQ_FORMAT_NVFP4>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    case DIALQ_FORMAT_MXFP4: return gemv_act<DIALQ_FORMAT_MXFP4>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    case DIALQ_FORMAT_Q4_K: return gemv_act<DIALQ_FORMAT_Q4_K>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
    case DIALQ_FORMAT_Q6_K: return gemv_act<DIALQ_FORMAT_Q6_K>(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, query, st, group);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const WeightView &w, const void *x, int x_dtype, int64_t M, void *y, int y_dtype, float *ws,
                       size_t ws_bytes, int *cnt, int *err, hipStream_t st) {
  return gemv_fmt(w, x, x_dtype, M, y, y_dtype, ws, ws_bytes, cnt, err, nullptr, st);
}

namespace {
std::atomic<int64_t> g_grouped_launches{0};
}

int64_t gemv_grouped_launches() { return g_grouped_launches.load(std::memory_order_relaxed); }

hipError_t launch_gemv_group(const WeightView *ws, void *const *ys, int n, const void *x, int x_dtype, int64_t M,
                             int y_dtype, hipStream_t st) {
  if (n < 2 || n > kGemvMaxGroup) return hipErrorNotSupported;
  GemvParams g{};
  g.w = ws[0];
  g.y = ys[0];
  g.nm = n;
  g.sbase[0] = 0;
  for (int j = 0; j < n; ++j) {
    if (ws[j].fmt != ws[0].fmt || ws[j].K != ws[0].K || ws[j].k_chunks != ws[0].k_chunks || ws[j].pair)
      return hipErrorNotSupported;
    g.wm[j] = ws[j];
    g.ym[j] = ys[j];
    g.sbase[j + 1] = g.sbase[j] + (int)ws[j].n_strips;
  }
  for (int j = n; j < kGemvMaxGroup; ++j) g.sbase[j + 1] = g.sbase[n];
  // a grouped launch never uses the workspace or the counters
  const hipError_t e = gemv_fmt(ws[0], x, x_dtype, M, ys[0], y_dtype, nullptr, 0, nullptr, nullptr, nullptr, st, &g);
  if (e == hipSuccess) g_grouped_launches.fetch_add(1, std::memory_order_relaxed);
  return e;
}

// The launch plan of launch_gemv, run without launching: the largest
// workspace any of its row-group launches takes (stream-K partials of equal
// tile ranges, or the work queue's piece partials; whole strips take none).
size_t gemv_workspace_bytes(const WeightView &w, int x_dtype, int64_t M) {
  size_t need = 0;
  if (M <= 0) return 0;
  if (gemv_fmt(w, nullptr, x_dtype, M, nullptr, DIALQ_BF16, nullptr, 0, nullptr, nullptr, &need, nullptr) != hipSuccess)
    return 0;
  return need;
}

}  // namespace dialq

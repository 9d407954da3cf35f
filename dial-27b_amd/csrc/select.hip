// Token selection after the lm_head, on the device.
//
// The reference samples the next token from one row of logits in
// sample_remote_logits (qwen3_vl/qwen3_vl.rs:282-323) through
// FastLogitsProcessor::sample (:130-174): greedy decoding with no repeat
// penalty takes candle's device argmax; otherwise the logits go to the host,
// the repeat penalty divides (logit >= 0) or multiplies (logit < 0) the logit
// of each distinct context token once (apply_repeat_penalty_in_place,
// :225-240), and ArgMax picks max_by(f32::total_cmp) -- the last of equal
// maxima -- while the sampling modes soften by the temperature
// (softmax_in_place, :325-345) and select the top-k / top-p candidates.
//
// Here the whole selection stays on the device and only k (index, logit)
// pairs and two statistics cross to the host:
//   1. k_select_slices: slice s of the vocabulary is converted to f32,
//      penalised and turned into 64-bit keys; for k = 1 the slice keeps its
//      largest key (a block max), otherwise chunks of up to 1024 / 2048 /
//      8192 keys (k <= 32 / 64 / above) join the k best carried so far and a block radix
//      select (block_topk) keeps the k best.  The slice's k best keys,
//      descending, and the (max, sum of exp(x - max)) of its
//      temperature-scaled logits go out;
//   2. k_select_merge: one workgroup stages the slices' lists in LDS (at
//      most 16384 keys, 128 KB), merges the statistics and radix-selects
//      the k best of all of them (a block max for k = 1), writing indices
//      and logits in descending order.
//
// Key of logit v at index i: the f32 bits mapped to an unsigned order
// (sign set: ~u, else u | 2^31), then the index in the low word:
//   rule 0 (candle argmax): -0 counts as +0, NaN below every number, ties
//          to the smaller index (low word ~i);
//   rule 1 (f32::total_cmp, Iterator::max_by): the IEEE total order, ties
//          to the larger index (low word i).
// Every real key is nonzero, so zero pads the partial slices and chunks.
#include "tile_ops.hpp"

namespace dialq {

constexpr int kSelMaxK = 256;          // largest k
constexpr int kSelMaxSlices = 1024;    // one statistics pair per thread of the merge
constexpr int kSelMaxKeys = 16384;     // slices x k staged by the merge: 128 KB of LDS

struct SelectParams {
  const void *logits;
  int dtype;
  int64_t vocab;
  const uint32_t *ids;  // distinct repeat-context tokens below vocab
  int n_ids;
  float penalty;        // 1: no penalty
  float temperature;    // > 0: also the softmax statistics of logits / temperature
  int rule;
  int slices;
  int64_t slice_len;
  int kc;               // carried keys per chunk (k)
  uint64_t *cand;       // [slices][k] keys, descending
  float *stats;         // [slices][2] (max, sum of exp(x - max)) of the scaled logits
  int k;
  uint32_t *out_idx;
  float *out_val;
  float *out_stats;     // (max, sum) over the vocabulary
};

__device__ __forceinline__ uint64_t select_key(float v, uint32_t idx, int rule) {
  uint32_t u = __float_as_uint(v);
  uint32_t key;
  if (rule == 0) {
    if (v != v) {
      key = 0u;
    } else {
      if (v == 0.0f) u = 0u;
      key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
  }
  key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  key = key < 1u ? 1u : key;  // keeps the all-ones NaN above the zero pad
  return ((uint64_t)key << 32) | (uint64_t)idx;
}

__device__ __forceinline__ float key_logit(uint64_t key) {
  const uint32_t k = (uint32_t)(key >> 32);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ uint32_t key_index(uint64_t key, int rule) {
  const uint32_t lo = (uint32_t)key;
  return rule == 0 ? 0xFFFFFFFFu - lo : lo;
}

// LDS scratch of block_topk.
struct TopkScratch {
  int hist[4 * 256];        // digit counts, one table per wave % 4
  int tot[256];
  uint64_t sel[kSelMaxK];   // the k keys, unordered
  uint64_t prefix, mask;
  int need, done, count;
};

// The k largest of n distinct keys in LDS, in descending order into out[0..k)
// (LDS; may alias keys), by the whole workgroup (NT threads).  Radix select
// on 8-bit digits from the top: each pass counts the digit of the keys that
// share the prefix chosen so far, and one wave finds the digit whose bucket
// holds the k-th largest.  It stops as soon as that bucket is needed whole
// (usually after two or three passes); then exactly k keys have their masked
// value at or above the prefix.  They are gathered and placed by rank
// (k <= 256: each thread counts the keys above its own).  Zero keys are
// padding below every real key; n must hold at least k real keys.
template <int NT>
__device__ __forceinline__ void block_topk(const uint64_t *keys, int n, int k, uint64_t *out, TopkScratch &sc) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) {
    sc.prefix = 0;
    sc.mask = 0;
    sc.need = k;
    sc.done = 0;
    sc.count = 0;
  }
  __syncthreads();
  for (int shift = 56; shift >= 0; shift -= 8) {
    if (sc.done) break;  // uniform: read after a barrier
    const uint64_t prefix = sc.prefix, mask = sc.mask;
    for (int i = tid; i < 4 * 256; i += NT) sc.hist[i] = 0;
    __syncthreads();
    int *h = sc.hist + (wave & 3) * 256;
    for (int i = tid; i < n; i += NT) {
      const uint64_t key = keys[i];
      if ((key & mask) == prefix) atomicAdd(&h[(key >> shift) & 255], 1);
    }
    __syncthreads();
    for (int d = tid; d < 256; d += NT) sc.tot[d] = sc.hist[d] + sc.hist[256 + d] + sc.hist[512 + d] + sc.hist[768 + d];
    __syncthreads();
    if (wave == 0) {
      // lane l holds digits 255 - 4l .. 252 - 4l (lane 0 the largest)
      int c[4], sum = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = sc.tot[255 - 4 * lane - j];
        sum += c[j];
      }
      int incl = sum;
      for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
      }
      const int excl = incl - sum, need = sc.need;
      if (excl < need && need <= incl) {  // exactly one lane
        int acc = excl, dj = 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= need) {
            dj = j;
            break;
          }
          acc += c[j];
        }
        const int rem = need - acc;
        sc.prefix = prefix | ((uint64_t)(255 - 4 * lane - dj) << shift);
        sc.mask = mask | ((uint64_t)0xFF << shift);
        sc.need = rem;
        sc.done = c[dj] == rem;
      }
    }
    __syncthreads();
  }
  const uint64_t prefix = sc.prefix, mask = sc.mask;
  for (int i = tid; i < n; i += NT) {
    const uint64_t key = keys[i];
    if ((key & mask) >= prefix) {
      const int slot = atomicAdd(&sc.count, 1);
      if (slot < kSelMaxK) sc.sel[slot] = key;
    }
  }
  __syncthreads();
  for (int t = tid; t < k; t += NT) {
    const uint64_t key = sc.sel[t];
    int r = 0;
    for (int j = 0; j < k; ++j) r += sc.sel[j] > key;
    out[r] = key;
  }
  __syncthreads();
}

// Sum (or max) of one value per thread over a 256-thread workgroup.
template <bool MAX>
__device__ __forceinline__ float block_reduce256(float v, float *sh) {
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off);
    v = MAX ? fmaxf(v, o) : v + o;
  }
  __syncthreads();  // sh free from the previous reduction
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return MAX ? fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3])) : (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// One DPP step of a wave max: each enabled lane takes the max of its key and
// the key of the lane CTRL names (row_shr:n = 0x110 + n, row_bcast:15 =
// 0x142, row_bcast:31 = 0x143); lanes without a source keep their own.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_step(uint64_t v) {
  const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
  const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xf, false);
  const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xf, false);
  const uint64_t o = ((uint64_t)ohi << 32) | olo;
  return o > v ? o : v;
}

// Max of a 64-bit key over the wave, in every lane: row_shr 1, 2, 4, 8 leave
// each 16-lane row's max in its lane 15, row_bcast 15 / 31 carry it into the
// rows above, and lane 63 ends with the wave's max.
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t v) {
  v = dpp_max_step<0x111, 0xf>(v);
  v = dpp_max_step<0x112, 0xf>(v);
  v = dpp_max_step<0x114, 0xf>(v);
  v = dpp_max_step<0x118, 0xf>(v);
  v = dpp_max_step<0x142, 0xa>(v);
  v = dpp_max_step<0x143, 0xc>(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

template <int C>
__global__ __launch_bounds__(256) void k_select_slices(SelectParams p) {
  __shared__ uint64_t keys[C];
  __shared__ float vals[C];
  __shared__ float sh[4];
  __shared__ uint64_t shk[4];
  __shared__ TopkScratch tsc;
  const int tid = threadIdx.x;
  const int kc = p.kc, payload = C - kc;
  const int64_t lo = (int64_t)blockIdx.x * p.slice_len;
  const int64_t hi = (lo + p.slice_len < p.vocab) ? lo + p.slice_len : p.vocab;
  for (int i = tid; i < kc; i += 256) keys[i] = 0;
  int carried = 0;  // real keys in keys[0..kc)
  float run_m = -INFINITY, run_s = 0.0f;
  const bool stats = p.temperature > 0.0f;
  for (int64_t base = lo; base < hi; base += payload) {
    const int n = (int)((hi - base) < payload ? (hi - base) : payload);
    for (int i = tid; i < n; i += 256) vals[i] = load_in(p.logits, base + i, p.dtype);
    __syncthreads();
    if (p.penalty != 1.0f) {
      for (int j = tid; j < p.n_ids; j += 256) {
        const int64_t id = p.ids[j];
        if (id >= base && id < base + n) {
          const float v = vals[id - base];
          vals[id - base] = v >= 0.0f ? v / p.penalty : v * p.penalty;
        }
      }
      __syncthreads();
    }
    if (stats) {
      float m = -INFINITY;
      for (int i = tid; i < n; i += 256) m = fmaxf(m, vals[i] / p.temperature);
      m = block_reduce256<true>(m, sh);
      // a chunk of -inf logits (a masked vocabulary range) adds exp(-inf) =
      // 0 to the sum, as softmax_in_place does; exp(v - m) would be
      // exp(-inf + inf) = NaN here.  m is the same in every thread.
      if (m != -INFINITY) {
        float sum = 0.0f;
        for (int i = tid; i < n; i += 256) sum += expf(vals[i] / p.temperature - m);
        sum = block_reduce256<false>(sum, sh);
        if (m > run_m) {
          run_s = run_s * expf(run_m - m) + sum;
          run_m = m;
        } else {
          run_s += sum * expf(m - run_m);
        }
      }
    }
    if (p.k == 1) {
      // the largest key of the chunk and the one carried
      uint64_t best = tid == 0 ? keys[0] : 0;
      for (int i = tid; i < n; i += 256) {
        const uint64_t key = select_key(vals[i], (uint32_t)(base + i), p.rule);
        best = key > best ? key : best;
      }
      best = wave_max_u64_dpp(best);
      if ((tid & 63) == 0) shk[tid >> 6] = best;
      __syncthreads();
      if (tid == 0) {
        uint64_t b = shk[0];
        for (int w = 1; w < 4; ++w) b = shk[w] > b ? shk[w] : b;
        keys[0] = b;
      }
      __syncthreads();
      continue;
    }
    for (int i = tid; i < n; i += 256) keys[kc + i] = select_key(vals[i], (uint32_t)(base + i), p.rule);
    __syncthreads();
    // the k best of the carried keys and this chunk's, back to keys[0..kk);
    // carried slots past the real keys hold zero pads
    const int kk = p.k < carried + n ? p.k : carried + n;
    block_topk<256>(keys, kc + n, kk, keys, tsc);
    for (int i = kk + tid; i < kc; i += 256) keys[i] = 0;
    carried = kk;
    __syncthreads();
  }
  uint64_t *out = p.cand + (size_t)blockIdx.x * p.k;
  for (int i = tid; i < p.k; i += 256) out[i] = keys[i];
  if (tid == 0) {
    p.stats[2 * blockIdx.x] = run_m;
    p.stats[2 * blockIdx.x + 1] = run_s;
  }
}

// Sum (or max) of one value per thread over a 1024-thread workgroup.
template <bool MAX>
__device__ __forceinline__ float block_reduce1024(float v, float *sh) {
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off);
    v = MAX ? fmaxf(v, o) : v + o;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
  for (int w = 1; w < 16; ++w) r = MAX ? fmaxf(r, sh[w]) : r + sh[w];
  return r;
}

__global__ __launch_bounds__(1024) void k_select_merge(SelectParams p) {
  extern __shared__ __attribute__((aligned(16))) uint64_t lists[];  // [slices][k]
  __shared__ float sh[16];
  __shared__ TopkScratch tsc;
  const int tid = threadIdx.x;
  const int G = p.slices, k = p.k;
  for (int i = tid; i < G * k; i += 1024) lists[i] = p.cand[i];
  // softmax statistics: max of the slice maxima, then their rescaled sums
  const float ms = tid < G ? p.stats[2 * tid] : -INFINITY, ss = tid < G ? p.stats[2 * tid + 1] : 0.0f;
  const float M = block_reduce1024<true>(ms, sh);
  const float S = block_reduce1024<false>(ss > 0.0f ? ss * expf(ms - M) : 0.0f, sh);
  if (tid == 0) {
    p.out_stats[0] = M;
    p.out_stats[1] = S;
  }
  __syncthreads();
  if (k == 1) {  // argmax: the largest of the slice maxima
    __shared__ uint64_t shk[16];
    const uint64_t best = wave_max_u64_dpp(tid < G ? lists[tid] : 0);
    if ((tid & 63) == 0) shk[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
      uint64_t b = shk[0];
      for (int w = 1; w < 16; ++w) b = shk[w] > b ? shk[w] : b;
      p.out_idx[0] = key_index(b, p.rule);
      p.out_val[0] = key_logit(b);
    }
    return;
  }
  // the k best of all slices' candidates (zero pads below every real key)
  block_topk<1024>(lists, G * k, k, lists, tsc);
  if (tid < k) {
    p.out_idx[tid] = key_index(lists[tid], p.rule);
    p.out_val[tid] = key_logit(lists[tid]);
  }
}

size_t select_workspace_bytes(int64_t vocab) {
  (void)vocab;
  return (size_t)kSelMaxKeys * sizeof(uint64_t) + (size_t)kSelMaxSlices * 2 * sizeof(float);
}

hipError_t launch_select(const void *logits, int dtype, int64_t vocab, const uint32_t *ids, int n_ids, float penalty,
                         float temperature, int rule, int k, void *ws, size_t ws_bytes, uint32_t *out_idx,
                         float *out_val, float *out_stats, hipStream_t st) {
  if (k < 1 || k > kSelMaxK || vocab < k || vocab > 0xFFFFFFFFLL || ws_bytes < select_workspace_bytes(vocab))
    return hipErrorInvalidValue;
  // chunk keys per slice step: a radix pass costs about the chunk (its
  // digit counts pile onto few bins), so small k takes short chunks and
  // many slices, large k long chunks so that slices x k fits the merge's
  // LDS; k = 1 keeps a running max.
  const int kc = k;
  const int C = k <= 32 ? 1024 : (k <= 64 ? 2048 : 8192);
  const int64_t cap = kSelMaxKeys / k < kSelMaxSlices ? kSelMaxKeys / k : kSelMaxSlices;
  int64_t g = (vocab + (C - kc) - 1) / (C - kc);
  if (g > cap) g = cap;
  SelectParams p;
  p.logits = logits;
  p.dtype = dtype;
  p.vocab = vocab;
  p.ids = ids;
  p.n_ids = n_ids;
  p.penalty = penalty;
  p.temperature = temperature;
  p.rule = rule;
  p.slices = (int)(g < 1 ? 1 : g);
  p.slice_len = (vocab + p.slices - 1) / p.slices;
  p.kc = kc;
  p.cand = (uint64_t *)ws;
  p.stats = (float *)((uint8_t *)ws + (size_t)kSelMaxKeys * sizeof(uint64_t));
  p.k = k;
  p.out_idx = out_idx;
  p.out_val = out_val;
  p.out_stats = out_stats;
  if (C == 1024) k_select_slices<1024><<<p.slices, 256, 0, st>>>(p);
  else if (C == 2048) k_select_slices<2048><<<p.slices, 256, 0, st>>>(p);
  else k_select_slices<8192><<<p.slices, 256, 0, st>>>(p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_select_merge<<<1, 1024, (size_t)p.slices * k * sizeof(uint64_t), st>>>(p);
  return hipGetLastError();
}

}  // namespace dialq

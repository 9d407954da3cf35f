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
//   1. k_select_slices: slice s of the vocabulary, in chunks of 3840 logits
//      behind the 256 best keys so far, is converted to f32, penalised, and
//      bitonic-sorted as 64-bit keys in LDS; the slice's 256 best keys and
//      the (max, sum of exp(x - max)) of its temperature-scaled logits go out;
//   2. k_select_merge: one workgroup loads every slice's keys into LDS
//      (at most 72 x 256 x 8 B = 144 KB), finds the k-th largest key by an
//      8-bit radix select over the 64-bit keys, gathers the k keys above it,
//      sorts them and writes indices and logits in descending order, plus
//      the merged softmax statistics.
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

constexpr int kSelKP = 256;           // keys kept per slice; the largest k
constexpr int kSelChunk = 4096;       // keys sorted per chunk step
constexpr int kSelPayload = kSelChunk - kSelKP;
constexpr int kSelMaxSlices = 72;     // 72 x 256 keys fill 144 KB of the merge's LDS

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
  uint64_t *cand;       // [slices][kSelKP] keys, descending
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

// Descending bitonic sort of n (a power of two) keys in LDS by the whole
// workgroup (nt threads).
__device__ __forceinline__ void bitonic_desc(uint64_t *keys, int n, int nt) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < n / 2; t += nt) {
        const int i = 2 * t - (t & (stride - 1)), l = i + stride;
        const uint64_t a = keys[i], b = keys[l];
        const bool first_half_desc = (i & size) == 0;
        if (first_half_desc ? (a < b) : (a > b)) {
          keys[i] = b;
          keys[l] = a;
        }
      }
      __syncthreads();
    }
  }
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

__global__ __launch_bounds__(256) void k_select_slices(SelectParams p) {
  __shared__ uint64_t keys[kSelChunk];
  __shared__ float vals[kSelPayload];
  __shared__ float sh[4];
  const int tid = threadIdx.x;
  const int64_t lo = (int64_t)blockIdx.x * p.slice_len;
  const int64_t hi = (lo + p.slice_len < p.vocab) ? lo + p.slice_len : p.vocab;
  for (int i = tid; i < kSelKP; i += 256) keys[i] = 0;
  float run_m = -INFINITY, run_s = 0.0f;
  const bool stats = p.temperature > 0.0f;
  for (int64_t base = lo; base < hi; base += kSelPayload) {
    const int n = (int)((hi - base) < kSelPayload ? (hi - base) : kSelPayload);
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
      float s = 0.0f;
      for (int i = tid; i < n; i += 256) s += expf(vals[i] / p.temperature - m);
      s = block_reduce256<false>(s, sh);
      if (m > run_m) {
        run_s = run_s * expf(run_m - m) + s;
        run_m = m;
      } else {
        run_s += s * expf(m - run_m);
      }
    }
    for (int i = tid; i < kSelPayload; i += 256)
      keys[kSelKP + i] = i < n ? select_key(vals[i], (uint32_t)(base + i), p.rule) : 0;
    __syncthreads();
    bitonic_desc(keys, kSelChunk, 256);
  }
  uint64_t *out = p.cand + (size_t)blockIdx.x * kSelKP;
  for (int i = tid; i < kSelKP; i += 256) out[i] = keys[i];
  if (tid == 0) {
    p.stats[2 * blockIdx.x] = run_m;
    p.stats[2 * blockIdx.x + 1] = run_s;
  }
}

__global__ __launch_bounds__(1024) void k_select_merge(SelectParams p) {
  extern __shared__ __attribute__((aligned(16))) uint64_t smem[];
  uint64_t *keys = smem;                                   // [slices * kSelKP]
  uint64_t *sel = smem + (size_t)p.slices * kSelKP;        // [kSelKP]
  int *hist = (int *)(sel + kSelKP);                       // [256]
  __shared__ uint64_t s_prefix;
  __shared__ int s_need, s_count;
  const int tid = threadIdx.x;
  const int n = p.slices * kSelKP;
  for (int i = tid; i < n; i += 1024) keys[i] = p.cand[i];
  if (tid < kSelKP) sel[tid] = 0;
  if (tid == 0) {
    float m = -INFINITY;
    for (int s = 0; s < p.slices; ++s) m = fmaxf(m, p.stats[2 * s]);
    float sum = 0.0f;
    for (int s = 0; s < p.slices; ++s)
      if (p.stats[2 * s + 1] > 0.0f) sum += p.stats[2 * s + 1] * expf(p.stats[2 * s] - m);
    p.out_stats[0] = m;
    p.out_stats[1] = sum;
    s_prefix = 0;
    s_need = p.k;
    s_count = 0;
  }
  __syncthreads();
  // 8-bit radix select of the k-th largest key (keys are distinct)
  uint64_t prefix = 0, mask = 0;
  for (int shift = 56; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += 1024) {
      const uint64_t key = keys[i];
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid == 0) {
      int need = s_need, cum = 0, d = 255;
      for (; d > 0; --d) {
        if (cum + hist[d] >= need) break;
        cum += hist[d];
      }
      s_need = need - cum;
      s_prefix = prefix | ((uint64_t)d << shift);
    }
    __syncthreads();
    prefix = s_prefix;
    mask |= (uint64_t)0xFF << shift;
  }
  // the k keys at or above the k-th largest
  for (int i = tid; i < n; i += 1024) {
    const uint64_t key = keys[i];
    if (key >= prefix) {
      const int slot = atomicAdd(&s_count, 1);
      if (slot < kSelKP) sel[slot] = key;
    }
  }
  __syncthreads();
  bitonic_desc(sel, kSelKP, 1024);
  if (tid < p.k) {
    p.out_idx[tid] = key_index(sel[tid], p.rule);
    p.out_val[tid] = key_logit(sel[tid]);
  }
}

size_t select_workspace_bytes(int64_t vocab) {
  const int64_t slices = select_slices(vocab);
  return (size_t)slices * kSelKP * sizeof(uint64_t) + (size_t)slices * 2 * sizeof(float);
}

int select_slices(int64_t vocab) {
  int64_t s = (vocab + kSelPayload - 1) / kSelPayload;
  if (s > kSelMaxSlices) s = kSelMaxSlices;
  return (int)(s < 1 ? 1 : s);
}

hipError_t launch_select(const void *logits, int dtype, int64_t vocab, const uint32_t *ids, int n_ids, float penalty,
                         float temperature, int rule, int k, void *ws, size_t ws_bytes, uint32_t *out_idx,
                         float *out_val, float *out_stats, hipStream_t st) {
  if (k < 1 || k > kSelKP || vocab < k || vocab > 0xFFFFFFFFLL || ws_bytes < select_workspace_bytes(vocab))
    return hipErrorInvalidValue;
  SelectParams p;
  p.logits = logits;
  p.dtype = dtype;
  p.vocab = vocab;
  p.ids = ids;
  p.n_ids = n_ids;
  p.penalty = penalty;
  p.temperature = temperature;
  p.rule = rule;
  p.slices = select_slices(vocab);
  p.slice_len = (vocab + p.slices - 1) / p.slices;
  p.cand = (uint64_t *)ws;
  p.stats = (float *)((uint8_t *)ws + (size_t)p.slices * kSelKP * sizeof(uint64_t));
  p.k = k;
  p.out_idx = out_idx;
  p.out_val = out_val;
  p.out_stats = out_stats;
  k_select_slices<<<p.slices, 256, 0, st>>>(p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds = (size_t)p.slices * kSelKP * 8 + kSelKP * 8 + 256 * 4;
  k_select_merge<<<1, 1024, lds, st>>>(p);
  return hipGetLastError();
}

}  // namespace dialq

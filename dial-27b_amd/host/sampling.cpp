// Remote token sampling with device-side selection (see sampling.hpp).
#include "sampling.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <string>

#include "dialq.h"

namespace dial {

namespace {

[[noreturn]] void fail(const std::string &msg) { throw Error(msg); }

inline uint32_t rotl(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

inline void quarter(uint32_t &a, uint32_t &b, uint32_t &c, uint32_t &d) {
  a += b; d ^= a; d = rotl(d, 16);
  c += d; b ^= c; b = rotl(b, 12);
  a += b; d ^= a; d = rotl(d, 8);
  c += d; b ^= c; b = rotl(b, 7);
}

thread_local bool t_used_host = false;

int dtype_code(DType t) {
  switch (t) {
    case DType::F32: return DIALQ_F32;
    case DType::F16: return DIALQ_F16;
    case DType::BF16: return DIALQ_BF16;
    default: fail(std::string("remote sampling takes F32, F16 or BF16 logits, got ") + dtype_name(t));
  }
}

float half_to_f32(uint16_t h, bool bf16) {
  if (bf16) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
  }
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else {  // subnormal: normalise
      int e = -1;
      uint32_t m = man;
      do {
        ++e;
        m <<= 1;
      } while (!(m & 0x400));
      u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ff) << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// logits_to_f32_vec (qwen3_vl.rs:240-255): the whole row on the host.
std::vector<float> host_logits(const Tensor &logits) {
  const std::vector<uint8_t> b = logits.host_bytes();
  const int64_t n = logits.elem_count();
  std::vector<float> out((size_t)n);
  if (logits.dtype() == DType::F32) {
    std::memcpy(out.data(), b.data(), (size_t)n * 4);
  } else {
    const bool bf = logits.dtype() == DType::BF16;
    for (int64_t i = 0; i < n; ++i) {
      uint16_t h;
      std::memcpy(&h, b.data() + 2 * i, 2);
      out[(size_t)i] = half_to_f32(h, bf);
    }
  }
  return out;
}

// apply_repeat_penalty_in_place (qwen3_vl.rs:225-240)
void repeat_penalty_host(std::vector<float> &logits, float penalty, const std::vector<uint32_t> &context) {
  std::vector<uint32_t> seen;
  for (uint32_t t : context) {
    if (std::find(seen.begin(), seen.end(), t) != seen.end()) continue;
    seen.push_back(t);
    if (t < logits.size()) {
      float &v = logits[t];
      v = v >= 0.0f ? v / penalty : v * penalty;
    }
  }
}

// softmax_in_place (qwen3_vl.rs:325-345)
void softmax_host(std::vector<float> &v, float temperature) {
  const float t = std::max(temperature, 1e-7f);
  float mx = -std::numeric_limits<float>::infinity();
  for (float &x : v) {
    x /= t;
    mx = std::fmax(mx, x);
  }
  float sum = 0.0f;
  for (float &x : v) {
    x = std::exp(x - mx);
    sum += x;
  }
  if (sum > 0.0f && std::isfinite(sum))
    for (float &x : v) x /= sum;
}

// f32::total_cmp as a signed order
int32_t total_key(float f) {
  int32_t i;
  std::memcpy(&i, &f, 4);
  return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// sample_topp's cut (qwen3_vl.rs:176-192): in descending order of
// probability, everything after the running sum reaches p becomes zero.
void topp_cut(std::vector<float> &prs, float p) {
  std::vector<uint32_t> idx(prs.size());
  for (size_t i = 0; i < idx.size(); ++i) idx[i] = (uint32_t)i;
  std::stable_sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) { return total_key(prs[a]) > total_key(prs[b]); });
  float cum = 0.0f;
  for (uint32_t i : idx) {
    if (cum >= p) prs[i] = 0.0f;
    else cum += prs[i];
  }
}

uint32_t topp_host(std::vector<float> &prs, float p, ChaChaRng &rng) {
  if (p > 0.0f && p < 1.0f) topp_cut(prs, p);
  return sample_weighted(prs, rng);
}

// Draw among candidates (token ids, probabilities) the way WeightedIndex
// draws over the whole probability vector in token order, in which the
// tokens left out weigh zero and add nothing to the cumulative sums.
uint32_t draw_in_token_order(std::vector<uint32_t> ids, std::vector<float> prs, ChaChaRng &rng) {
  std::vector<size_t> ord(ids.size());
  for (size_t i = 0; i < ord.size(); ++i) ord[i] = i;
  std::sort(ord.begin(), ord.end(), [&](size_t a, size_t b) { return ids[a] < ids[b]; });
  std::vector<float> w(ord.size());
  std::vector<uint32_t> t(ord.size());
  for (size_t i = 0; i < ord.size(); ++i) {
    w[i] = prs[ord[i]];
    t[i] = ids[ord[i]];
  }
  return t[sample_weighted(w, rng)];
}

// The reference's host path over the whole vocabulary.
uint32_t sample_on_host(const Tensor &logits, const SamplingRequest &req, int mode, ChaChaRng &rng) {
  t_used_host = true;
  std::vector<float> v = host_logits(logits);
  if (req.repeat_penalty != 1.0f) repeat_penalty_host(v, req.repeat_penalty, req.repeat_context);
  if (mode == 0) {
    size_t best = 0;
    for (size_t i = 1; i < v.size(); ++i)
      if (total_key(v[i]) >= total_key(v[best])) best = i;
    if (v.empty()) fail("empty logits");
    return (uint32_t)best;
  }
  softmax_host(v, (float)req.temperature);
  if (mode == 1) return sample_weighted(v, rng);
  const uint64_t k = req.top_k.value_or(0);
  const float p = (float)req.top_p.value_or(1.0);
  if (mode == 3) return topp_host(v, p, rng);
  if (k >= v.size()) return mode == 2 ? sample_weighted(v, rng) : topp_host(v, p, rng);
  // select_nth_unstable_by(k, descending): the k best.  The reference then
  // draws in the order that partition leaves them, which Rust does not
  // specify; here they are drawn in token order.
  std::vector<uint32_t> idx(v.size());
  for (size_t i = 0; i < idx.size(); ++i) idx[i] = (uint32_t)i;
  std::stable_sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) { return total_key(v[a]) > total_key(v[b]); });
  std::vector<float> top((size_t)k);
  for (uint64_t i = 0; i < k; ++i) top[i] = v[idx[i]];
  if (mode == 4 && p > 0.0f && p < 1.0f) topp_cut(top, p);
  idx.resize((size_t)k);
  return draw_in_token_order(idx, top, rng);
}

// The selection's workspace and output buffers, one grow-only pair per
// device, reused by every sampled token: allocating them per token would
// add hipMalloc / hipFree round trips (and hipFree's device-wide wait) to
// each token's 7-75 us selection.
struct SelectBuffers {
  std::mutex mu;
  Tensor ws, out;
};

SelectBuffers &select_buffers(int device) {
  static std::mutex m;
  static std::map<int, std::unique_ptr<SelectBuffers>> all;
  std::lock_guard<std::mutex> lk(m);
  std::unique_ptr<SelectBuffers> &b = all[device];
  if (!b) b = std::make_unique<SelectBuffers>();
  return *b;
}

struct DeviceSelection {
  std::vector<uint32_t> idx;
  std::vector<float> val;
  float m = 0.0f, s = 0.0f;
};

DeviceSelection select_on_device(const Tensor &logits, int64_t vocab, const SamplingRequest &req, float temperature,
                                 int rule, int64_t k) {
  DeviceSelection r;
  r.idx.resize((size_t)k);
  r.val.resize((size_t)k);
  float st[2];
  char err[512];
  const bool dev = logits.device().is_rocm();
  const uint32_t *ids = req.repeat_context.empty() ? nullptr : req.repeat_context.data();
  // host logits go up once; the selection's outputs come back in one copy
  const int device = dev ? logits.device().ordinal : 0;
  const void *lp = logits.data();
  Tensor dlog;
  if (!dev) {
    dlog = logits.to_device(Device::rocm(0));
    lp = dlog.data();
  }
  const size_t wsb = dialq_logits_select_workspace_bytes(vocab, (int64_t)req.repeat_context.size());
  SelectBuffers &buf = select_buffers(device);
  std::lock_guard<std::mutex> lk(buf.mu);  // one selection at a time per device owns the buffers
  if (!buf.ws.defined() || buf.ws.nbytes() < wsb) buf.ws = Tensor::empty(DType::U8, {(int64_t)wsb}, Device::rocm(device));
  if (!buf.out.defined())
    buf.out = Tensor::empty(DType::U8, {(int64_t)(8 * DIALQ_SELECT_MAX_K + 8)}, Device::rocm(device));
  Tensor &ws = buf.ws, &out = buf.out;
  uint32_t *oi = (uint32_t *)out.data();
  float *ov = (float *)((uint8_t *)out.data() + 4 * k), *os = (float *)((uint8_t *)out.data() + 8 * k);
  if (dialq_logits_select(lp, dtype_code(logits.dtype()), vocab, ids, (int64_t)req.repeat_context.size(),
                          req.repeat_penalty, temperature, rule, k, oi, ov, os, ws.data(), wsb, device, nullptr, 1,
                          err, sizeof err) != 0)
    fail(std::string("remote sampling failed: ") + err);
  // synchronous: waits for the selection (2 KB: the buffer holds 256 candidates)
  const std::vector<uint8_t> hb = out.host_bytes();
  std::memcpy(r.idx.data(), hb.data(), 4 * (size_t)k);
  std::memcpy(r.val.data(), hb.data() + 4 * k, 4 * (size_t)k);
  std::memcpy(st, hb.data() + 8 * k, 8);
  r.m = st[0];
  r.s = st[1];
  return r;
}

constexpr int64_t kMaxDeviceK = DIALQ_SELECT_MAX_K;

}  // namespace

// ---- generator ---------------------------------------------------------------
std::array<uint32_t, 16> ChaChaRng::block(const std::array<uint32_t, 8> &key, uint32_t counter,
                                          const std::array<uint32_t, 3> &nonce, int rounds) {
  std::array<uint32_t, 16> in = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, key[0], key[1], key[2], key[3],
                                 key[4],      key[5],      key[6],      key[7],      counter, nonce[0], nonce[1],
                                 nonce[2]};
  std::array<uint32_t, 16> x = in;
  for (int r = 0; r < rounds; r += 2) {
    quarter(x[0], x[4], x[8], x[12]);
    quarter(x[1], x[5], x[9], x[13]);
    quarter(x[2], x[6], x[10], x[14]);
    quarter(x[3], x[7], x[11], x[15]);
    quarter(x[0], x[5], x[10], x[15]);
    quarter(x[1], x[6], x[11], x[12]);
    quarter(x[2], x[7], x[8], x[13]);
    quarter(x[3], x[4], x[9], x[14]);
  }
  for (int i = 0; i < 16; ++i) x[i] += in[i];
  return x;
}

ChaChaRng ChaChaRng::seed_from_u64(uint64_t state) {
  std::array<uint32_t, 8> key;
  for (int i = 0; i < 8; ++i) {
    state = state * 6364136223846793005ull + 11634580027462260723ull;
    const uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    const uint32_t rot = (uint32_t)(state >> 59);
    key[i] = (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
  }
  return ChaChaRng(key, 12);
}

uint32_t ChaChaRng::next_u32() {
  if (pos_ >= 16) {
    // 64-bit block counter in words 12-13, stream id 0 in words 14-15
    buf_ = block(key_, (uint32_t)counter_, {(uint32_t)(counter_ >> 32), 0u, 0u}, rounds_);
    ++counter_;
    pos_ = 0;
  }
  return buf_[pos_++];
}

uint32_t sample_weighted(const std::vector<float> &weights, ChaChaRng &rng) {
  if (weights.empty()) fail("weighted sampling failed: No weights provided in distribution");
  std::vector<float> cumulative;
  cumulative.reserve(weights.size());
  float total = 0.0f;
  for (size_t i = 0; i < weights.size(); ++i) {
    const float w = weights[i];
    if (!(w >= 0.0f) || !std::isfinite(w)) fail("weighted sampling failed: A weight is invalid in distribution");
    if (i > 0) cumulative.push_back(total);
    total += w;
  }
  if (!(total > 0.0f)) fail("weighted sampling failed: All weights are zero in distribution");
  if (!std::isfinite(total)) fail("weighted sampling failed: Too many weights (hint: try reducing them)");
  // UniformFloat<f32>::new(0, total): scale shrinks until the largest draw stays below total
  const float max_rand = 1.0f - std::numeric_limits<float>::epsilon();
  float scale = total;
  while (scale * max_rand + 0.0f >= total) scale = std::nextafter(scale, 0.0f);
  const uint32_t bits = (rng.next_u32() >> 9) | 0x3f800000u;
  float v12;
  std::memcpy(&v12, &bits, 4);
  const float chosen = (v12 - 1.0f) * scale + 0.0f;
  // partition_point(|w| w <= chosen) over the cumulative weights before each item
  size_t lo = 0, hi = cumulative.size();
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cumulative[mid] <= chosen) lo = mid + 1;
    else hi = mid;
  }
  return (uint32_t)lo;
}

int sampling_mode(const SamplingRequest &req) {
  if (req.temperature <= 0.0) return 0;
  if (!req.top_k && !req.top_p) return 1;
  if (req.top_k && !req.top_p) return 2;
  if (!req.top_k) return 3;
  return 4;
}

bool last_sample_used_host_logits() { return t_used_host; }

uint32_t sample_remote_logits(const Tensor &logits, const SamplingRequest &req) {
  t_used_host = false;
  const std::vector<int64_t> &d = logits.dims();
  int64_t vocab;
  if (d.size() == 1) vocab = d[0];
  else if (d.size() == 2 && d[0] == 1) vocab = d[1];
  else fail("remote sampling failed: remote sampling expects [vocab] or [1, vocab] logits, got " + logits.dims_debug());
  if (vocab < 1) fail("remote sampling failed: empty logits");
  const uint64_t seed = req.seed ^ (req.sample_index * 0x9E3779B97F4A7C15ull);
  ChaChaRng rng = ChaChaRng::seed_from_u64(seed);
  const int mode = sampling_mode(req);
  if (mode == 0) {
    // greedy: candle's device argmax, or max_by(total_cmp) after the penalty
    const bool pen = req.repeat_penalty != 1.0f;
    return select_on_device(logits, vocab, req, 0.0f, pen ? DIALQ_SELECT_TOTAL_LAST_MAX : DIALQ_SELECT_FIRST_MAX, 1)
        .idx[0];
  }
  const float t = std::max((float)req.temperature, 1e-7f);
  const uint64_t k = req.top_k.value_or(0);
  const float p = (float)req.top_p.value_or(1.0);
  if (mode == 1 || ((mode == 2 || mode == 4) && (k >= (uint64_t)vocab || k > (uint64_t)kMaxDeviceK)) ||
      (mode == 2 && k == 0))
    return sample_on_host(logits, req, mode, rng);
  if (mode == 3 && (p <= 0.0f || p >= 1.0f)) return sample_on_host(logits, req, mode, rng);
  const int64_t kk = (mode == 3) ? std::min<int64_t>(kMaxDeviceK, vocab) : (int64_t)k;
  const DeviceSelection sel = select_on_device(logits, vocab, req, t, DIALQ_SELECT_TOTAL_LAST_MAX, kk);
  // softmax_in_place's probabilities of the candidates (descending)
  std::vector<float> prs((size_t)kk);
  for (int64_t i = 0; i < kk; ++i) prs[(size_t)i] = std::exp(sel.val[(size_t)i] / t - sel.m) / sel.s;
  if (mode == 2) return draw_in_token_order(sel.idx, prs, rng);
  if (mode == 4) {
    if (p > 0.0f && p < 1.0f) topp_cut(prs, p);
    return draw_in_token_order(sel.idx, prs, rng);
  }
  // TopP: the nucleus must close inside the device's candidates
  float cum = 0.0f;
  int64_t keep = 0;
  for (; keep < kk && cum < p; ++keep) cum += prs[(size_t)keep];
  if (cum < p && kk < vocab) return sample_on_host(logits, req, mode, rng);
  std::vector<uint32_t> ids(sel.idx.begin(), sel.idx.begin() + keep);
  prs.resize((size_t)keep);
  return draw_in_token_order(ids, prs, rng);
}

}  // namespace dial

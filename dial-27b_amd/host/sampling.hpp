// Remote token sampling after the output head, with the selection on the
// device (dialq_logits_select).
//
// Mirrors sample_remote_logits (qwen3_vl/qwen3_vl.rs:282-323), which the
// GGUF worker calls when --worker-gguf-sample-token is set
// (qwen3_vl/worker_gguf.rs:366-383), and FastLogitsProcessor::sample
// (:130-174) beneath it:
//   * seed ^ sample_index * 0x9E3779B97F4A7C15 seeds a fresh generator per
//     token; temperature <= 0 is ArgMax, otherwise All / TopK / TopP /
//     TopKThenTopP by which of top_k, top_p are set;
//   * ArgMax without a repeat penalty is the device argmax (candle's rule:
//     ties to the first index); with a penalty, max_by(f32::total_cmp) over
//     the penalised logits (ties to the last index);
//   * the sampling modes take the k <= 256 best candidates and the softmax
//     normaliser from the device, so the probability of candidate i is
//     exp(logit_i / t - M) / S as softmax_in_place computes it; TopP keeps
//     candidates while the running sum is below p. When the request needs
//     more than 256 candidates (top_k > 256, a nucleus that the 256 best do
//     not close, or plain multinomial sampling over the whole vocabulary) the
//     logits are copied to the host and the reference's own host steps run.
//
// The generator restates rand 0.9's StdRng (ChaCha12, seeded through
// rand_core's PCG32 seed_from_u64) and WeightedIndex<f32> (cumulative sums,
// UniformFloat in [0, total), partition_point).  rand is a third-party crate
// absent from the reference tree: the random draw is parity unpinned; the
// ChaCha block function is checked against RFC 7539's test vector.
#pragma once

#include <array>
#include <cstdint>
#include <optional>
#include <vector>

#include "dial_host.hpp"

namespace dial {

// spm/proto/message.rs:184-192
struct SamplingRequest {
  uint64_t seed = 0;
  uint64_t sample_index = 0;
  double temperature = 0.0;
  std::optional<uint64_t> top_k;
  std::optional<double> top_p;
  float repeat_penalty = 1.0f;
  std::vector<uint32_t> repeat_context;
};

// rand 0.9 StdRng: ChaCha with 12 rounds, 64-bit block counter, stream 0.
class ChaChaRng {
 public:
  explicit ChaChaRng(const std::array<uint32_t, 8> &key, int rounds = 12) : key_(key), rounds_(rounds) {}
  static ChaChaRng seed_from_u64(uint64_t state);  // rand_core's PCG32 expansion
  uint32_t next_u32();
  // One 64-byte block for (key, counter, nonce words 13..15) -- the RFC 7539
  // layout when counter < 2^32 -- exposed for the known-answer test.
  static std::array<uint32_t, 16> block(const std::array<uint32_t, 8> &key, uint32_t counter,
                                        const std::array<uint32_t, 3> &nonce, int rounds);

 private:
  std::array<uint32_t, 8> key_;
  int rounds_;
  uint64_t counter_ = 0;
  std::array<uint32_t, 16> buf_{};
  int pos_ = 16;
};

// WeightedIndex<f32>::new(weights).sample(rng): errors like the reference
// ("weighted sampling failed: ...") on empty, negative, non-finite or
// all-zero weights.
uint32_t sample_weighted(const std::vector<float> &weights, ChaChaRng &rng);

// The sampling mode the reference takes for a request (0 ArgMax, 1 All,
// 2 TopK, 3 TopP, 4 TopKThenTopP) and whether the last call of
// sample_remote_logits in this thread read the whole vocabulary on the host.
int sampling_mode(const SamplingRequest &req);
bool last_sample_used_host_logits();

// sample_remote_logits: logits [vocab] or [1, vocab] (F32 / F16 / BF16, on a
// ROCm device or the host).
uint32_t sample_remote_logits(const Tensor &logits, const SamplingRequest &req);

}  // namespace dial

// K2 entry: path sampling (Gumbel-max) and the dispatch to path replay
// (sample_replay.hip) and to the reference causal sampler (sample_ref.hip).
#include "sample_impl.h"

namespace ta {

hipError_t launch_sample(const Plan& P, const void* q, const float* U, uint64_t seed, float* weights,
                         char* rec, hipStream_t st, const uint8_t* paths) {
  if (P.p.causal == TA_CAUSAL_REFERENCE) return launch_ref_sample(P, q, U, seed, weights, rec, st);
  if (paths) return launch_sample_replay(P, q, weights, rec, st, paths);
  return sample_dispatch<false>(P, q, U, seed, weights, rec, st, nullptr);
}

TA_SAMPLE_TYPED(false, bf16)

}  // namespace ta

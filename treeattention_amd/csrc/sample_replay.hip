// Path replay: the sampler's kernels with every decision taken from packed
// path bits (sample_impl.h, kReplay = true).
#include "sample_impl.h"

namespace ta {

hipError_t launch_sample_replay(const Plan& P, const void* q, float* weights, char* rec, hipStream_t st,
                                const uint8_t* paths) {
  return sample_dispatch<true>(P, q, nullptr, 0, weights, rec, st, paths);
}

TA_SAMPLE_TYPED(true, bf16)

}  // namespace ta

// K2: path replay, fp16 inputs (sample_impl.h), a translation unit of its own so the
// sampler's instantiations compile in parallel.
#include "sample_impl.h"

namespace ta {

TA_SAMPLE_TYPED(true, f16)

}  // namespace ta

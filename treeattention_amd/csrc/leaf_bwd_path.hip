// The leaf backward with the tree gradient of every pair's sampled path
// (leaf_bwd_tr_kernel with 16 or 32 path rows, leaf_bwd_tr.h), in a
// translation unit of its own so it compiles beside leaf_bwd.hip.
#include "leaf_bwd_tr.h"

namespace ta {

// (make_plan gives no path rows to tiles that do not fit the LDS)
template <typename E, int D, int LBP>
static hipError_t path_lbp(const Plan& P, const LeafBwdArgs& a, unsigned grid, hipStream_t st) {
  if constexpr (BwdTrTile<D, LBP, 16>::bytes <= 160 * 1024) {
    if (P.path_rows == 16) return launch_bwd_tr<E, D, LBP, 16>(a, grid, st);
  }
  if constexpr (BwdTrTile<D, LBP, 32>::bytes <= 160 * 1024) {
    if (P.path_rows == 32) return launch_bwd_tr<E, D, LBP, 32>(a, grid, st);
  }
  return hipErrorInvalidValue;
}

template <typename E, int D>
static hipError_t path_d(const Plan& P, const LeafBwdArgs& a, unsigned grid, hipStream_t st) {
  switch (padded_keys(P.geo.LB)) {
    case 32: return path_lbp<E, D, 32>(P, a, grid, st);
    case 64: return path_lbp<E, D, 64>(P, a, grid, st);
    default: return path_lbp<E, D, 128>(P, a, grid, st);
  }
}

template <typename E>
static hipError_t path_e(const Plan& P, const LeafBwdArgs& a, unsigned grid, hipStream_t st) {
  switch (P.D) {
    case 32: return path_d<E, 32>(P, a, grid, st);
    case 64: return path_d<E, 64>(P, a, grid, st);
    case 96: return path_d<E, 96>(P, a, grid, st);
    default: return path_d<E, 128>(P, a, grid, st);
  }
}

hipError_t launch_leaf_bwd_path(const Plan& P, const LeafBwdArgs& a, unsigned grid, hipStream_t st) {
  switch (P.p.dtype) {
    case TA_BF16: return path_e<bf16>(P, a, grid, st);
    case TA_F16: return path_e<f16>(P, a, grid, st);
    default: return hipErrorInvalidValue;  // 16-bit inputs only
  }
}

}  // namespace ta

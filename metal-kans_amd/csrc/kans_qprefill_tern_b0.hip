// Fused prefill kernels of one weight format (tern) without the base
// branch: the instantiations of kan_qfused_block (kans_qprefill_kernel.h)
// that qp_supported lists.
#include "kans_qprefill_kernel.h"

namespace kans {

hipError_t qp_run_tern_b0(const QPLaunch& L, const QPGrid& G, hipStream_t st) { return qp_run<Q_TERN, 0>(L, G, st); }

}  // namespace kans

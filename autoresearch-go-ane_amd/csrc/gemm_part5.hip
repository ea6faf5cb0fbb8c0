// Instantiates the GEMM launchers of group 5 of gemm_launchers.inc (split
// over several files so that the kernels compile in parallel).
#include "gemm_impl.h"

namespace ane {
namespace gemm_detail {
#define ANE_GEMM_LAUNCH(AT, BT, E) \
  template hipError_t launch<AT, BT, E>(const GemmArgs&, const EpiParams&, hipStream_t, int, int, int, int);
#define ANE_GEMM_G1(AT, BT, E)
#define ANE_GEMM_G2(AT, BT, E)
#define ANE_GEMM_G3(AT, BT, E)
#define ANE_GEMM_G4(AT, BT, E)
#define ANE_GEMM_G5 ANE_GEMM_LAUNCH
#include "gemm_launchers.inc"
}  // namespace gemm_detail
}  // namespace ane

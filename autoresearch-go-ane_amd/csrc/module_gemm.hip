// The forward's GEMM kernels under C names, for the code object a host
// loads itself (hipModuleLoad, ../../include/ane_kernels.h).  Each entry
// point is one instantiation of the hand-ordered kernel libane_hip.so
// launches for the llama2 eval forward (the deferred-norm form), with its
// arguments as the library passes them; compiled only into ane_gemm.hsaco.
#include <cstddef>

#include "../../include/ane_kernels.h"
#include "gemm_impl.h"

namespace ane {
namespace gemm_detail {

// The C structs of the header lay out exactly as the kernels' own.
#define ANE_SAME_FIELD(C, CPP, F) static_assert(offsetof(C, F) == offsetof(CPP, F), #C "." #F)
static_assert(sizeof(AneGemmArgs) == sizeof(GemmArgs) && sizeof(AneEpiParams) == sizeof(EpiParams),
              "argument struct sizes");
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, A);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, ldb);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, K);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, a_t);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, b_t);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, grp);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, b_group_stride);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, splits);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, ws);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, pf);
ANE_SAME_FIELD(AneGemmArgs, GemmArgs, pf_bytes);
ANE_SAME_FIELD(AneEpiParams, EpiParams, ldc);
ANE_SAME_FIELD(AneEpiParams, EpiParams, C2);
ANE_SAME_FIELD(AneEpiParams, EpiParams, R);
ANE_SAME_FIELD(AneEpiParams, EpiParams, scale);
ANE_SAME_FIELD(AneEpiParams, EpiParams, beta_ptr);
ANE_SAME_FIELD(AneEpiParams, EpiParams, seq);
ANE_SAME_FIELD(AneEpiParams, EpiParams, targets);
ANE_SAME_FIELD(AneEpiParams, EpiParams, tgt_logit);
ANE_SAME_FIELD(AneEpiParams, EpiParams, softcap);
ANE_SAME_FIELD(AneEpiParams, EpiParams, cap);
ANE_SAME_FIELD(AneEpiParams, EpiParams, vocab);
ANE_SAME_FIELD(AneEpiParams, EpiParams, C3);
ANE_SAME_FIELD(AneEpiParams, EpiParams, gain);
ANE_SAME_FIELD(AneEpiParams, EpiParams, ssq_part);
ANE_SAME_FIELD(AneEpiParams, EpiParams, ssq_ld);
ANE_SAME_FIELD(AneEpiParams, EpiParams, rr_part);
ANE_SAME_FIELD(AneEpiParams, EpiParams, rr_ld);
ANE_SAME_FIELD(AneEpiParams, EpiParams, rr_dim);
#undef ANE_SAME_FIELD

extern "C" __global__ __launch_bounds__(256) void ane_k_gemm_qkv_rr(GemmArgs g, EpiParams e) {
  gemm_ho_body<128, 192, EPI_STORE_H_RR, 4>(g, e);
}
extern "C" __global__ __launch_bounds__(256) void ane_k_gemm_resid_norm(GemmArgs g, EpiParams e) {
  gemm_ho_body<128, 64, EPI_RESID_NORM, 4>(g, e);
}
extern "C" __global__ __launch_bounds__(512) void ane_k_gemm_swiglu_rr(GemmArgs g, EpiParams e) {
  gemm_ho_body<256, 256, EPI_SWIGLU_RR, 8>(g, e);
}
extern "C" __global__ __launch_bounds__(512) void ane_k_gemm_ce_rr(GemmArgs g, EpiParams e) {
  gemm_ho_body<256, 256, EPI_CE_RR, 8>(g, e);
}

}  // namespace gemm_detail
}  // namespace ane

// Explicit instantiation of the GLA backward launch sequence for one
// (dtype, head dim, decay form), chosen by HOFA_INST_DT / HOFA_INST_D /
// HOFA_INST_GEN (0: log_gamma [* alpha], 1: general g) on the compile line.
// The build compiles this file once per (dtype, head dim) pair listed in
// HOFA_GLA_BWD_FOR_EACH and per decay form, so the heavy chunk kernels build
// in parallel.
#include "hofa_gla_bwd_kernels.h"

#if !defined(HOFA_INST_DT) || !defined(HOFA_INST_D) || !defined(HOFA_INST_GEN)
#error "compile with -DHOFA_INST_DT=<HOFA_F32|HOFA_BF16|HOFA_F16> -DHOFA_INST_D=<64|128> -DHOFA_INST_GEN=<0|1>"
#endif

namespace hofa {
namespace glabwd {
template int launch_d<HOFA_INST_DT, HOFA_INST_D, (HOFA_INST_GEN != 0)>(const GlaBwdK &, int, hipStream_t);
}  // namespace glabwd
}  // namespace hofa

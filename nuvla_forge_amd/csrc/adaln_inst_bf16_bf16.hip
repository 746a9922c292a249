// adaLN row kernels instantiated for x = bf16, y = bf16.
#include "adaln_impl.h"

namespace nf {
namespace adaln {
template int fwd_v<bf16, bf16>(const FwdArgs &, const Plan &, bool, hipStream_t);
template int bwd_v<bf16, bf16>(const BwdArgs &, const Plan &, bool, hipStream_t);
}  // namespace adaln
}  // namespace nf

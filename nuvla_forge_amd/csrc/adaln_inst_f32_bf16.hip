// adaLN row kernels instantiated for x = float, y = bf16.
#include "adaln_impl.h"

namespace nf {
namespace adaln {
template int fwd_v<float, bf16>(const FwdArgs &, const Plan &, bool, hipStream_t);
template int bwd_v<float, bf16>(const BwdArgs &, const Plan &, bool, hipStream_t);
}  // namespace adaln
}  // namespace nf

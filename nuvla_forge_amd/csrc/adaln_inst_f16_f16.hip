// adaLN row kernels instantiated for x = f16, y = f16.
#include "adaln_impl.h"

namespace nf {
namespace adaln {
template int fwd_v<f16, f16>(const FwdArgs &, const Plan &, bool, hipStream_t);
template int bwd_v<f16, f16>(const BwdArgs &, const Plan &, bool, hipStream_t);
}  // namespace adaln
}  // namespace nf

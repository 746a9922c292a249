// adaLN row kernels instantiated for x = float, y = float.
#include "adaln_impl.h"

namespace nf {
namespace adaln {
template int fwd_v<float, float>(const FwdArgs &, const Plan &, bool, hipStream_t);
template int bwd_v<float, float>(const BwdArgs &, const Plan &, bool, hipStream_t);
}  // namespace adaln
}  // namespace nf

// Backward eval3d compositing variants for the colour dimensions of XSG_CDIM_GROUP7.
#include "eval3d_bwd_kernel.h"

namespace xsg {
#define XSG_INST(C) template int eval3d_bwd_cdim<C>(bool, bool, const Eval3dParams&, hipStream_t);
XSG_CDIM_GROUP7(XSG_INST)
#undef XSG_INST
}  // namespace xsg

// Backward eval3d compositing: dispatch on the colour dimension to the per-CDIM launchers that
// eval3d_bwd_g<k>.hip instantiate from eval3d_bwd_kernel.h.
#include "xsg_eval3d.h"

namespace xsg {

int eval3d_bwd_launch(int cdim, bool dyn, const Eval3dParams& p, hipStream_t s) {
    const bool ray_grads = p.v_ray_o != nullptr;
    switch (cdim) {
#define XSG_CASE(C) case C: return eval3d_bwd_cdim<C>(dyn, ray_grads, p, s);
        XSG_CDIM_LIST(XSG_CASE)
#undef XSG_CASE
        default: return xsg_fail(XSG_ERR_INVALID, "unsupported feature dimension: %d", cdim);
    }
}

}  // namespace xsg

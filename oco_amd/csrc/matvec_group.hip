// The grouped streaming matvec: several matrices of one format and shape
// over the same activation rows in one grid (oco_matvec_group), so that
// the projections that share an input -- ffn_gate and ffn_up after one
// norm -- stream back to back without a launch between them, with the
// activation vector (and its fused norm) staged once per workgroup for all
// of them.  The reference issues the second of such a pair with
// apply_norm_concurrent, which skips the barrier between the two dispatches
// (src/weights/compute/feed_forward.rs:97-104, compute/matrix.rs:127-146,
// src/gpu/dispatch.rs:235-259).  The kernel is stream_kernel with MULTI set.
#include "stream_kernel.h"

namespace oco {

StreamFn stream_pick_group(bool x_bf16, uint32_t fmt, int xs, int npl, bool direct, int &lpr) {
    return x_bf16 ? stream_pick_format<bf16_t, true>(fmt, xs, npl, direct, lpr)
                  : stream_pick_format<float, true>(fmt, xs, npl, direct, lpr);
}

}  // namespace oco

// MFMA (gfx950 matrix core) variants of the fused tensor-ring kernel.
#include "trk_internal.h"

namespace trk {

int mfma_register(Plan *plan) {
    (void)plan;
    return 0;
}

}  // namespace trk

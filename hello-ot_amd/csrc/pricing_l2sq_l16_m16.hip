// l2^2 pricing scan driver instantiated for partial lists of 16 entries merged into the best 16 per row.
#include "l2sq_impl.h"

namespace hm {
int l2sq_run_l16_m16(L2SQ_RUN_ARGS) { return run_bidir<16, 16>(L2SQ_RUN_PASS); }
}  // namespace hm

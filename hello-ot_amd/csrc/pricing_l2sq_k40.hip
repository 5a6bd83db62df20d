// l2^2 pricing scan driver instantiated for per-lane lists of 40 entries.
#include "l2sq_impl.h"

namespace hm {
int l2sq_run_k40(L2SQ_RUN_ARGS) { return run_bidir<40>(L2SQ_RUN_PASS); }
}  // namespace hm

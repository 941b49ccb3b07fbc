// The persistent denoise kernel for batches of kRowSplitMinBatch and more
// (denoise_loop_kernel<true, 2>: row-split gate_up; grouped attention from kAttnGroupMinBatch on),
// compiled in a translation unit of its own so that no instance's code generation depends on
// another's.
#define PI05_PERSISTENT_INSTANCE 2
#include "pi05_persistent.hip"

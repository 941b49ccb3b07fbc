// The persistent denoise kernel for batches of 2 (denoise_loop_kernel<true, 1>), compiled in a
// translation unit of its own so that no instance's code generation depends on another's.
#define PI05_PERSISTENT_INSTANCE 1
#include "pi05_persistent.hip"

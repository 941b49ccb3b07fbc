// The batched instance of the persistent denoise kernel (denoise_loop_kernel<true>), compiled in a
// translation unit of its own so that neither instance's code generation depends on the other's.
#define PI05_PERSISTENT_INSTANCE 1
#include "pi05_persistent.hip"

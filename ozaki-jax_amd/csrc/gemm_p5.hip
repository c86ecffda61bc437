// The host schedules' instantiations: launch_ap_host, one of the parts
// gemm.hip dispatches to.
#define OZK_GEMM_PART 5
#define OZK_GEMM_PART_HOST 1
#include "gemm.hip"

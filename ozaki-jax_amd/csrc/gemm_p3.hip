// Part 3 of the all-pairs schedules' instantiations (gemm_parts.h).
#include "gemm_parts.h"
#define OZK_GEMM_PART 3
#define OZK_GEMM_PART_FN launch_ap_part3
#define OZK_GEMM_PART_TUPLES OZK_GEMM_PART3_TUPLES
#include "gemm.hip"

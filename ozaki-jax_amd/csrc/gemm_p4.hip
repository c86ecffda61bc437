// Part 4 of the all-pairs schedules' instantiations (gemm_parts.h).
#include "gemm_parts.h"
#define OZK_GEMM_PART 4
#define OZK_GEMM_PART_FN launch_ap_part4
#define OZK_GEMM_PART_TUPLES OZK_GEMM_PART4_TUPLES
#include "gemm.hip"

// Part 2 of the all-pairs schedules' instantiations (gemm_parts.h).
#include "gemm_parts.h"
#define OZK_GEMM_PART 2
#define OZK_GEMM_PART_FN launch_ap_part2
#define OZK_GEMM_PART_TUPLES OZK_GEMM_PART2_TUPLES
#include "gemm.hip"

// Part 1 of the all-pairs schedules' instantiations (gemm_parts.h).
#include "gemm_parts.h"
#define OZK_GEMM_PART 1
#define OZK_GEMM_PART_FN launch_ap_part1
#define OZK_GEMM_PART_TUPLES OZK_GEMM_PART1_TUPLES
#include "gemm.hip"

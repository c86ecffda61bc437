// Part 2 of the rectangle sweeps' instantiations (gemm_parts.h).
#include "gemm_parts.h"
#define OZK_GEMM_PART 7
#define OZK_GEMM_PART_RECT 1
#define OZK_GEMM_PART_FN launch_ap_rect2
#define OZK_GEMM_RECT_SHAPES OZK_GEMM_RECT2_SHAPES
#include "gemm.hip"

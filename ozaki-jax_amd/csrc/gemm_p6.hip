// Part 1 of the rectangle sweeps' instantiations (gemm_parts.h).
#include "gemm_parts.h"
#define OZK_GEMM_PART 6
#define OZK_GEMM_PART_RECT 1
#define OZK_GEMM_PART_FN launch_ap_rect1
#define OZK_GEMM_RECT_SHAPES OZK_GEMM_RECT1_SHAPES
#include "gemm.hip"

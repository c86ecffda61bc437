// The (n_hi, n_lo) all-pairs schedules instantiated in the parts of
// gemm.hip (gemm_p1.hip .. gemm_p4.hip), one translation unit each so that
// they compile in parallel; gemm.hip itself holds the presets and (1,1),
// (2,1), (2,2).
#pragma once
#define OZK_GEMM_PART1_TUPLES(X) X(5, 1) X(5, 2) X(5, 3) X(1, 2) X(1, 3)
#define OZK_GEMM_PART2_TUPLES(X) X(5, 5) X(4, 5) X(4, 3) X(1, 4) X(2, 3)
#define OZK_GEMM_PART3_TUPLES(X) X(3, 5) X(3, 4) X(2, 5) X(1, 5) X(3, 2)
#define OZK_GEMM_PART4_TUPLES(X) X(4, 2) X(2, 4) X(4, 4) X(3, 3)

// The (n_hi, n_lo) all-pairs schedules instantiated in the parts of
// gemm.hip (gemm_p1.hip .. gemm_p4.hip), one translation unit each so that
// they compile in parallel; gemm.hip itself holds the presets and (1,1),
// (2,1), (2,2).
#pragma once
#define OZK_GEMM_PART1_TUPLES(X) X(5, 1) X(5, 2) X(5, 3) X(1, 2) X(1, 3)
#define OZK_GEMM_PART2_TUPLES(X) X(5, 5) X(4, 5) X(4, 3) X(1, 4) X(2, 3)
#define OZK_GEMM_PART3_TUPLES(X) X(3, 5) X(3, 4) X(2, 5) X(1, 5) X(3, 2)
#define OZK_GEMM_PART4_TUPLES(X) X(4, 2) X(2, 4) X(4, 4) X(3, 3)

// The (NA, NB) shapes of the rectangle sweeps (every on-device schedule
// with both counts up to 8 that has no fixed sweeps), in gemm_p6.hip and
// gemm_p7.hip.
#define OZK_GEMM_RECT1_SHAPES(X)                                                      \
  X(1, 1) X(1, 7) X(2, 2) X(2, 7) X(2, 8) X(3, 3) X(3, 4) X(3, 5) X(3, 6) X(3, 7)   \
  X(5, 5) X(6, 2) X(7, 3) X(8, 1)
#define OZK_GEMM_RECT2_SHAPES(X)                                                      \
  X(1, 6) X(1, 8) X(2, 6) X(4, 3) X(4, 4) X(4, 5) X(4, 6) X(6, 1) X(6, 3) X(6, 4)   \
  X(7, 1) X(7, 2) X(8, 2)

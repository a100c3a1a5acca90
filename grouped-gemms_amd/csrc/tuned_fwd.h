// Tuned forward launch configurations, one per swept shape, consulted by
// pick_fwd (grouped_gemm.hip) before its built-in rule.  Written by
// `python grouped-gemms_amd/tune_driver.py --emit-header` from the sweep's
// best.json; regenerate rather than edit.  An entry applies to calls with
// the same E, N, K and weight format and M within a factor of two of the
// swept M, on every operand layout (the sweep timed the drop-in call's,
// operands staged by the library's rule at the swept shape; the whole entry
// applies elsewhere too, since the tile order can change the bits of a call
// whose last round is split).  Fields: E, M, N, K, b_fmt (0 e4m3, 4 e2m1),
// block_m, block_n,
// group_m, xcd swizzle, split (1: the last round may be split along K when
// the workspace allows it, 0: whole tiles only).
// sweep: 36 shapes (e4m3, 8 offset draws), 18 with a gain of at least 1% on every draw; AMD Radeon Graphics
static const TunedFwd kTunedFwd[] = {
    {1, 16640, 2048, 2048, 0, 256, 256, 1, 8, 1},   // 88.8 us
    {1, 16640, 2048, 5120, 0, 256, 256, 4, 1, 1},   // 176.9 us
    {1, 16640, 2048, 8192, 0, 256, 256, 4, 1, 1},   // 251.3 us
    {1, 16640, 5120, 2048, 0, 256, 256, 12, 8, 0},   // 187.9 us
    {1, 16640, 5120, 5120, 0, 256, 256, 4, 1, 1},   // 401.5 us
    {1, 16640, 5120, 8192, 0, 256, 256, 4, 1, 1},   // 615.6 us
    {1, 16640, 8192, 2048, 0, 256, 256, 1, 1, 1},   // 275.7 us
    {1, 16640, 8192, 5120, 0, 256, 256, 4, 8, 1},   // 596.8 us
    {1, 16640, 8192, 8192, 0, 256, 256, 1, 1, 1},   // 915.7 us
    {2, 16640, 2048, 2048, 0, 256, 256, 1, 8, 0},   // 90.7 us
    {2, 16640, 2048, 5120, 0, 256, 256, 4, 1, 1},   // 186.2 us
    {2, 16640, 2048, 8192, 0, 256, 256, 4, 1, 1},   // 266.1 us
    {2, 16640, 5120, 5120, 0, 256, 256, 4, 1, 1},   // 420.5 us
    {2, 16640, 8192, 2048, 0, 256, 256, 1, 1, 1},   // 284.4 us
    {4, 16640, 2048, 2048, 0, 256, 256, 1, 8, 0},   // 91.0 us
    {4, 16640, 8192, 5120, 0, 256, 256, 1, 1, 1},   // 638.0 us
    {4, 16640, 8192, 8192, 0, 256, 256, 1, 1, 1},   // 990.5 us
    {8, 16640, 8192, 2048, 0, 256, 256, 1, 1, 1},   // 291.2 us
    {0, 0, 0, 0, 0, 0, 0, 0, 0, 0},   // end
};

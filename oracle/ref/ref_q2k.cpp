// Test infrastructure: compiles ggml's stock AVX2 Q2_K x Q8_K dot, as the
// reference keeps it in bench/q2k_dot_bench.cpp:31-63, straight from the
// reference tree (the include path points there; nothing is copied).  The
// bench's own main() is renamed so this translation unit can be a library.
#define main zmref_q2k_bench_main
#include "q2k_dot_bench.cpp"
#undef main

extern "C" float zmref_dot_q2_K(int n, const void *x, const void *y) {
  return dot_stock(n, static_cast<const block_q2_K *>(x), static_cast<const block_q8_K *>(y));
}

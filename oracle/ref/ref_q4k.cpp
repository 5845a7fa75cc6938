// Test infrastructure: compiles the reference's 512-bit Q4_K x Q8_K dot
// (bench/q3k_q4k_dot_bench.cpp:73-125, stated there to be bit-exact with
// ggml's stock kernel) straight from the reference tree.  The bench's main()
// becomes an unused static function, so the ggml symbols only it references
// (the stock dots, absent here) are never emitted.
#define main static zmref_q34_bench_main
#include "q3k_q4k_dot_bench.cpp"
#undef main

extern "C" float zmref_dot_q4_K(int n, const void *x, const void *y) {
  return dot_q4k_512(n, static_cast<const block_q4_K *>(x), static_cast<const block_q8_K *>(y));
}

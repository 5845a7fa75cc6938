/* The members of ggml's public `struct ggml_tensor` that the adapter reads
 * (type, ne, nb, data), in a struct of that name, for compiling the adapter
 * in this repository's tests without a ggml checkout.  A real build compiles
 * the adapter against ggml's own ggml.h. */
#pragma once
#include <stddef.h>
#include <stdint.h>

enum ggml_type { GGML_TYPE_F32 = 0, GGML_TYPE_Q2_K = 10, GGML_TYPE_Q3_K = 11, GGML_TYPE_Q4_K = 12, GGML_TYPE_I32 = 26 };

struct ggml_tensor {
  enum ggml_type type;
  int64_t ne[4];
  size_t nb[4];
  void *data;
};

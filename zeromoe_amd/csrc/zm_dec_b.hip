// zm_dec_b.hip -- instantiations of the fused decode kernel (zm_decode.hpp) for Q2_K layers with and without a Q4_K shared expert, and the mixed
// K-quant layers of real checkpoints (Q4_K / Q5_K gate and up with a Q6_K down projection), IQ4_XS and IQ3_XXS layers.
#include "zm_decode.hpp"

namespace zm {

DecFn find_decode_b(int tg, int td, int ts, int l1, int ir, int is) {
  if (tg == T_Q2_K && td == T_Q2_K && ts == T_Q4_K) return dec_pick<T_Q2_K, T_Q2_K, T_Q4_K>(l1, ir, is);
  if (tg == T_Q2_K && td == T_Q2_K && ts == 0) return dec_pick<T_Q2_K, T_Q2_K, 0>(l1, ir, is);
  if (tg == T_Q4_K && td == T_Q6_K && ts == 0) return dec_pick<T_Q4_K, T_Q6_K, 0>(l1, ir, is);
  if (tg == T_Q5_K && td == T_Q6_K && ts == 0) return dec_pick<T_Q5_K, T_Q6_K, 0>(l1, ir, is);
  if (tg == T_IQ4_XS && td == T_IQ4_XS && ts == 0) return dec_pick<T_IQ4_XS, T_IQ4_XS, 0>(l1, ir, is);
  if (tg == T_IQ3_XXS && td == T_IQ3_XXS && ts == 0) return dec_pick<T_IQ3_XXS, T_IQ3_XXS, 0>(l1, ir, is);
  return nullptr;
}

}  // namespace zm

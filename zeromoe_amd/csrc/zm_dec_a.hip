// zm_dec_a.hip -- instantiations of the fused decode kernel (zm_decode.hpp) for the single-type layers of the benchmark configurations (Q4_K, Q2_K+Q3_K, IQ2_XXS).
#include "zm_decode.hpp"

namespace zm {

DecFn find_decode_a(int tg, int td, int ts, int l1, int ir, int is) {
  if (tg == T_Q4_K && td == T_Q4_K && ts == 0) return dec_pick<T_Q4_K, T_Q4_K, 0>(l1, ir, is);
  if (tg == T_Q2_K && td == T_Q3_K && ts == 0) return dec_pick<T_Q2_K, T_Q3_K, 0>(l1, ir, is);
  if (tg == T_IQ2_XXS && td == T_IQ2_XXS && ts == 0) return dec_pick<T_IQ2_XXS, T_IQ2_XXS, 0>(l1, ir, is);
  return nullptr;
}

}  // namespace zm

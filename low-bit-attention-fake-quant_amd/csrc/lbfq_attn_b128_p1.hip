// Instantiations of the attention kernel with block_n = 128 for P quant mode
// 1 (0 elementwise, 1 mx, 2 dynamic); split per mode so the translation
// units build in parallel.
#include "lbfq_attn_kernel.h"

namespace lbfq_attn {
int launch_b128_p1(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st) {
  return launch_p<1, 128>(a, D, qk_mx, rb, bl, valpha, st);
}
}  // namespace lbfq_attn

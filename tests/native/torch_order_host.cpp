// Host build of csrc/klc_torch_order.h for the CPU tests: the same
// sequential libstdc++ restatement and SLEEF expf the router kernel runs.
#include <stdint.h>

#include "klc_torch_order.h"

extern "C" {

// torch.topk order of one row of bfloat16 logits (n <= 65535; k - 1 <= 33)
void host_torch_topk(const uint16_t* row, int n, int k, int32_t* out, uint32_t* work) {
  for (int p = 0; p < n; ++p) work[p] = klc::order_entry(row[p], p);
  klc::torch_topk_order(work, n, k);
  for (int j = 0; j < k; ++j) out[j] = (int32_t)(work[j] & 0xffffu);
}

void host_sleef_expf(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = klc::sleef_expf_u10(x[i]);
}

}

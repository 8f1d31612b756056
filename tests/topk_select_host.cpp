// Host build of the router's selection routines (csrc/topk_select.h), so the
// CPU tests can check the kernel's selection order against torch.topk without
// a GPU.  rows x n probabilities in, rows x k indices out.
#include <stdint.h>

#include <vector>

#include "topk_select.h"

namespace {
struct ArrayQueue {
  da::topk::Entry* q;
  da::topk::Entry get(int i) const { return q[i]; }
  void set(int i, da::topk::Entry x) { q[i] = x; }
  void swap(int i, int j) {
    const da::topk::Entry t = q[i];
    q[i] = q[j];
    q[j] = t;
  }
};
}  // namespace

extern "C" void topk_rows(const float* probs, int64_t rows, int n, int k, int64_t* out) {
  std::vector<da::topk::Entry> buf(n);
  for (int64_t r = 0; r < rows; ++r) {
    for (int i = 0; i < n; ++i) buf[i] = {probs[r * n + i], i};
    ArrayQueue q{buf.data()};
    da::topk::select_topk(q, n, k);
    for (int s = 0; s < k; ++s) out[r * k + s] = buf[s].e;
  }
}

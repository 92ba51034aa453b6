// The head-dim-256 prefill kernel (prefill.hip) in a translation unit of its
// own: it is compiled with the max-ilp scheduling strategy, which the
// head-dim-64/128 kernels do not take (see the build's per-source flags).
#define XATTN_PREFILL_D256 1
#include "prefill.hip"

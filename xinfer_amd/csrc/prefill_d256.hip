// The head-dim-256 prefill kernel (prefill.hip) in a translation unit of its
// own, so that it takes its own scheduling strategy (max-ilp; the
// head-dim-64/128 kernels are faster with another, see the build's
// per-source flags).
#define XATTN_PREFILL_D256 1
#include "prefill.hip"

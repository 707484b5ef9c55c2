// q6k_short.hip -- the Q6_K instantiations of the short-team long-row
// K-split kernels (q4k_short.hip holds the Q4_K ones), compiled apart so the
// two build in parallel.
#define Q4K_SHORT_Q6 1
#include "q4k_short.hip"

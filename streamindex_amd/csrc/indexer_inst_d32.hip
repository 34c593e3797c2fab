// Instantiates the lightning-indexer kernels for head dim D_I = 32
// (32-head blocks 1, 2: H_I up to 64).
#include "indexer_launch.h"

namespace si {
SI_INSTANTIATE_INDEXER(1, 32)
SI_INSTANTIATE_INDEXER(2, 32)
}  // namespace si

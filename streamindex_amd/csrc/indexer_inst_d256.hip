// Instantiates the lightning-indexer kernels for head dim D_I = 256
// (32-head blocks 1, 2: H_I up to 64).
#include "indexer_launch.h"

namespace si {
SI_INSTANTIATE_INDEXER(1, 256)
SI_INSTANTIATE_INDEXER(2, 256)
}  // namespace si

// Instantiates the lightning-indexer kernels for head dim D_I = 32
// (32-head blocks 3, 4: H_I up to 128).
#include "indexer_launch.h"

namespace si {
SI_INSTANTIATE_INDEXER(3, 32)
SI_INSTANTIATE_INDEXER(4, 32)
}  // namespace si

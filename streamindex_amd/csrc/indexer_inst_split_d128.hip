// Instantiates the head-split top-k kernel (indexer_topk_split.h) for head
// dim D_I = 128: two waves per query row holding 1, 2 or 4 32-head blocks
// each (H_I up to 256), selection capacities 1536 and 4608.
#include "indexer_topk_split.h"

namespace si {
#define SI_INST_SPLIT(hs, hbh, d, c) template int launch_topk_split<hs, hbh, d, c>(const IndexerArgs&, hipStream_t);
SI_INST_SPLIT(2, 1, 128, 4608)
SI_INST_SPLIT(2, 2, 128, 4608)
SI_INST_SPLIT(2, 4, 128, 1536)
SI_INST_SPLIT(2, 4, 128, 4608)
#undef SI_INST_SPLIT
}  // namespace si

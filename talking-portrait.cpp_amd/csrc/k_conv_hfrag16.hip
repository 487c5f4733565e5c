// Halo convs with IC = 512 (16 chunks of 32 channels): the kernel
// instances of tpmd_hfrag.h, in a translation unit of their own.
#include "tpmd_hfrag.h"

namespace tpmd {

TPMD_HFRAG_NC(16);

}  // namespace tpmd

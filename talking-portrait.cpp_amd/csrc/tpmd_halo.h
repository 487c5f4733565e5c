// Constants of the halo convs (k_conv_hfrag.hip, k_conv_hfrag_tail.hip):
// the input halo of each 32-channel chunk sits in LDS with 80-byte pixels (4
// chunks of 8 channels + a pad chunk, so 32 consecutive pixels read at any
// offset hit distinct banks).
#pragma once

#include "tpmd_conv.h"

namespace tpmd {

constexpr int HR_PXB = 80;              // halo pixel: 64 bytes of channels + 16-byte pad
constexpr int HR_HBUF = 32 * 1024;      // one halo buffer: 32 units of 1 KB per wave-set

}  // namespace tpmd

// SPDX-License-Identifier: MIT
// Head dims of FLASH_ATTN_EXT: shared by the launcher and the placement rules.
#pragma once

namespace mx {

// The attention kernels are built for (DK, DV) = (64, 64), (128, 128), (192, 128) and
// (256, 256). Other head dims run on the smallest of them that holds both, zero-padded: Q and K
// columns past dk and V columns past dv read as zero (they add nothing to Q.K or to P.V), output
// columns past dv are not written. So every dk and dv up to 256 that are multiples of 8 are taken.
inline bool fa_pad_dims(int dk, int dv, int & D, int & DV) {
    static const int kDims[4][2] = {{64, 64}, {128, 128}, {192, 128}, {256, 256}};
    if (dk <= 0 || dv <= 0 || dk % 8 || dv % 8) return false;
    for (const auto & p : kDims)
        if (dk <= p[0] && dv <= p[1]) {
            D = p[0];
            DV = p[1];
            return true;
        }
    return false;
}

// Head dims past those builds (the absorbed MLA's 576 / 512) run as two GEMMs around a softmax
// pass (mx_fa_wide.hip): dk % 32 == 0 (the Q.K GEMM's depth), dv % 8 == 0, both up to 1024.
inline bool fa_wide_dims(int dk, int dv) {
    return dk > 0 && dv > 0 && dk % 32 == 0 && dv % 8 == 0 && dk <= 1024 && dv <= 1024;
}

}  // namespace mx

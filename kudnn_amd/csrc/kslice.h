// The forms of the f32 k-slice kernel (gemm_kslice.hip) that the planner needs to know about.
#ifndef KUDNN_KSLICE_H
#define KUDNN_KSLICE_H

#include <cstdint>

// Whether K takes the kernel's whole-line form (8 waves, whole 128-byte lines through a per-wave LDS tile): K = 256 c
// for c = 1, 2, 3, 4, 6, 8, 12 or 16. Only that form reads an fp32 weight stored [K][N] in place.
inline bool kudnn_kslice_whole_line(int64_t K)
{
    if (K <= 0 || K % 256 != 0) {
        return false;
    }
    switch (K / 256) {
        case 1: case 2: case 3: case 4: case 6: case 8: case 12: case 16: return true;
        default: return false;
    }
}

#endif  // KUDNN_KSLICE_H

// rlq_dtype.hpp - the GGML numeric type table (crates/quant/src/lib.rs:132-285):
// which ids exist, elements per block and bytes per block.  Host code only.
#pragma once

#include <stdint.h>

namespace rlq {

inline bool dtype_known(uint32_t id) {
    switch (id) {
        case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 9: case 10: case 11: case 12: case 13:
        case 14: case 15: case 16: case 17: case 18: case 19: case 20: case 21: case 22: case 23: case 24:
        case 25: case 26: case 27: case 28: case 29: case 30: case 34: case 35: case 39: case 40: case 41:
        case 42: case 43:
            return true;
        default:
            return false;
    }
}

inline uint64_t block_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 30: case 28: case 24: case 25: case 26: case 27: case 43: return 1;
        case 2: case 3: case 6: case 7: case 8: case 9: case 20: case 39: return 32;
        case 40: case 42: return 64;
        case 41: return 128;
        default: return 256;
    }
}

inline uint64_t type_size(uint32_t t) {
    switch (t) {
        case 0: case 26: return 4;
        case 1: case 30: case 25: return 2;
        case 28: case 27: return 8;
        case 24: case 43: return 1;
        case 2: case 20: case 41: case 42: return 18;
        case 3: return 20;
        case 6: return 22;
        case 7: return 24;
        case 8: return 34;
        case 9: case 40: return 36;
        case 10: return 84;
        case 11: return 110;
        case 12: return 144;
        case 13: return 176;
        case 14: return 210;
        case 15: return 292;
        case 16: case 35: return 66;
        case 17: return 74;
        case 18: return 98;
        case 19: return 50;
        case 21: return 110;
        case 22: return 82;
        case 23: return 136;
        case 29: return 56;
        case 34: return 54;
        case 39: return 17;
        default: return 0;
    }
}

}  // namespace rlq

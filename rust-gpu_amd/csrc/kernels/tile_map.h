// tile_map.h -- the integer maps that place tiles on workgroups and 16-byte
// chunks in LDS.  Plain integer code, inline for the device and for the
// host alike, so that the CPU tests run these very functions over whole
// index ranges (tests/test_tile_maps.py): a map that were not a bijection
// would compute some output tiles twice and others never, or read operand
// chunks from the wrong LDS slot.
#pragma once
#include <stdint.h>

#ifdef __HIPCC__
#define T0_HD __host__ __device__ inline
#else
#define T0_HD inline
#endif

namespace t0 {

// ------------------------------------------------------------- tile order --
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on
// XCD b % 8).  Remap so that consecutive logical ids share an XCD (and its
// L2): XCD x owns the contiguous id range [start(x), start(x) + count(x)).
T0_HD uint32_t xcd_remap(uint32_t b, uint32_t total) {
    const uint32_t NX = 8;
    uint32_t x = b % NX, i = b / NX;
    uint32_t q = total / NX, r = total % NX;
    uint32_t start = x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q;
    return start + i;
}

// Grouped (super-tile) order: GROUP_M tile rows are walked column by column
// so a run of consecutive ids covers a GROUP_M x (run/GROUP_M) block.
T0_HD void grouped_tile(uint32_t id, uint32_t tiles_m, uint32_t tiles_n, uint32_t group_m,
                        uint32_t& tm, uint32_t& tn) {
    uint32_t per_group = group_m * tiles_n;
    uint32_t g = id / per_group;
    uint32_t first_m = g * group_m;
    uint32_t gm = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
    uint32_t in = id - g * per_group;
    tm = first_m + in % gm;
    tn = in / gm;
}

// Swizzle for row-major [rows][CH chunks of 16 B] tiles read 16 lanes x 16 B
// at a time along rows (A, and B in NT form).
template <int CH>
T0_HD uint32_t swz_rows(uint32_t r) {
    if constexpr (CH >= 8) return ((r & 7) ^ ((r >> 3) & 1)) & (CH - 1);
    else if constexpr (CH == 4) return ((r >> 1) ^ (r >> 3)) & 3;
    else return ((r >> 2) ^ (r >> 3)) & 1;
}

// Swizzle for the NN B tile [BK][CHB chunks]: the transposed reads take four
// consecutive k rows x 32 B per 16-lane group.
template <int CHB>
T0_HD uint32_t swz_nn(uint32_t r) {
    return (0xEA40u >> ((r & 3) * 4)) & 0xFu & (CHB - 1);   // rows 0..3 -> 0, 4, 10, 14
}

}  // namespace t0

// mfma_tiles.h — which (expert, token tile, weight-row tile) a block of the
// matrix-core expert kernels computes, and the grids that cover them.
#pragma once
#include <hip/hip_runtime.h>

#include "moe_internal.h"

namespace moe {

// Tile coordinates.  mode 0: routed tiles from the dispatch list; mode 1: the
// shared expert over all T tokens.  The grid is walked in the order
// (expert, N tile, M tile), M fastest, and each XCD (linear block id mod 8)
// takes a contiguous range of that order: an expert's weight tile is read
// from HBM once and met in L2 by the expert's other M tiles, and the
// expert's activations stay in that XCD's L2 while its N tiles go by.
//
// A block holds a CU (its LDS ring fills it), so an XCD's range runs in
// rounds of xcd_cus blocks, and the last round is partly filled when the
// range is not a multiple of that.  When it would hold at most half a
// round of tiles (single-part launches), each of those last tiles is split
// in two blocks along its tokens: SUB-token subtiles [0, ceil(MT / 2)) in
// one and the rest in the other, at the end of the XCD's range, so the last
// round is full and each of its blocks does about half a tile's products.
// KHALF: the last tiles are split along K instead (khalf 0: the first half
// of the steps, 1: the rest), each such tile with a slot of its own (XCD
// x's i-th: x * kTailPerXcd + i) where the two blocks meet.
struct TileInfo {
    int g, m0, n, row0, ntile, ksplit;
    bool shared;
    int khalf = -1, slot = 0;
};
template <int BM, int SUB, bool KHALF = false>
__device__ inline bool tile_of(const MfmaArgs &a, int mode, int gx, TileInfo &ti) {
    const int gy = gridDim.y, gz = gridDim.z;
    const int total = gx * gy;
    const int lin = blockIdx.x + gx * blockIdx.y;
    ti.ksplit = gz > 1 ? (int)blockIdx.z : 0;
    const int mt_sh = (a.T + BM - 1) / BM;
    // Routed tiles come first in the tile list, the shared expert's last; a
    // launch walks only its own (at most gx of them, so valid <= total).
    const int valid = mode == 1 ? mt_sh * gy : (a.ntiles[0] - a.shared_tiles) * gy;
    // XCD x (= lin mod 8) takes t in [x * per, (x + 1) * per) in order.
    int t = lin, half = -1;
    if ((total & 7) == 0) {
        const int per = (valid + 7) >> 3;
        const int j = lin >> 3;
        const int tail = gz == 1 && a.xcd_cus > 0 ? per % a.xcd_cus : 0;
        if (tail > 0 && 2 * tail <= a.xcd_cus && 8 * (per + tail) <= total &&
            (!KHALF || (tail <= kTailPerXcd && a.tail_part && a.tail_cnt))) {
            // Blocks head .. head + tail - 1 take the first halves of the
            // XCD's last `tail` tiles, the next `tail` blocks their second.
            const int head = per - tail;
            if (j >= per + tail) return false;
            if (j < head) {
                t = (lin & 7) * per + j;
            } else {
                half = j - head >= tail;
                t = (lin & 7) * per + head + (j - head - (half ? tail : 0));
                if (KHALF) ti.khalf = half, ti.slot = (lin & 7) * kTailPerXcd + (j - head - (half ? tail : 0));
            }
        } else {
            if (j >= per) return false;
            t = (lin & 7) * per + j;
        }
    }
    if (t >= valid) return false;
    if (mode == 1) {
        ti.ntile = t / mt_sh;
        ti.g = a.E, ti.m0 = (t % mt_sh) * BM, ti.n = a.T, ti.row0 = 0, ti.shared = true;
    } else {
        // Tiles of one group are contiguous: t / gy lies inside t's group.
        const int ie = t / gy;
        const int f = a.tiles[4 * ie + 2], mt = a.tiles[4 * ie + 3];
        const int local = t - f * gy;
        const int i = f + local % mt;
        ti.ntile = local / mt;
        const int g = a.tiles[4 * i];
        if (g >= a.E) return false;
        ti.g = g, ti.m0 = a.tiles[4 * i + 1], ti.n = a.counts[g], ti.row0 = a.offsets[g], ti.shared = false;
    }
    if (half >= 0 && !KHALF) {
        // The tile's tokens [m0, end), end - m0 <= BM, in two parts.
        const int end = min(ti.n, ti.m0 + BM);
        const int mh = (end - ti.m0 + 2 * SUB - 1) / (2 * SUB);  // ceil(MT / 2) subtiles
        if (half == 0) {
            ti.n = min(end, ti.m0 + SUB * mh);
        } else {
            ti.m0 += SUB * mh;
            ti.n = end;
            if (ti.m0 >= end) return false;
        }
    }
    return true;
}

// CUs of the current device (256 when the query fails).
int device_cus();
// CUs per XCD for tile_of's split of the last round, or 0 (no split) when
// the tiles hold about `min_tokens` tokens or fewer: their second halves
// would be nearly empty blocks.
int split_cus(double tokens_per_tile, double min_tokens);
// Grid for `tiles` tile columns of `rows` weight rows in tiles of `cols`.
// With the split of the last round (xcd_cus > 0, one K part): room for it
// (half a round per XCD) and a multiple of 8 blocks, so the XCD order
// applies; `order` makes it apply where the plain grid would not be a
// multiple of 8.
dim3 tile_grid(int tiles, int rows, int cols, int ks, int xcd_cus, bool order);

}  // namespace moe

// Row plan of one 64-row tile, shared by the forward's row_plan kernel and the selection's
// sel_norms launch (which can compute the plan alongside the norms).
//
// Head-independent preparation read by the forward and dQ kernels.  Within each 64-row
// tile the rows are ordered by window start lo_i (ties by row; rows past the end last), so
// the 16 rows a wave takes have close window starts: the wave's key range [min lo, max i]
// and its count of masked subtiles shrink.  Each 16-row group's {min lo, max lo, max i,
// min i} is recorded, with the tile's largest clamped window (whose maximum over a sequence
// bounds the key-parallel backward sweep).
#pragma once

#include "common.h"

namespace dsalt {

struct PlanOut {
    uint8_t* perm;   // [S * n_tiles * 64] row offset within the tile
    int* bounds;     // [S * n_tiles * 4 * 4]
    int* wmax;       // [S * n_tiles]
};

// One wave (lane l) plans tile `tile` (= s * n_tiles + t) when `active`; sp, slo: 64 ints
// of LDS each, private to the wave.  Every thread of the block must call it once (one
// block barrier inside); nothing is written for an inactive tile.
__device__ __forceinline__ void row_plan_tile(const int32_t* w, const int32_t* cu, int total_len, int max_seqlen,
                                              int n_tiles, int tile, bool active, int l, int* sp, int* slo,
                                              const PlanOut& o) {
    const int s = active ? tile / n_tiles : 0, t = active ? tile % n_tiles : 0;
    int st = 0, len = 0;
    if (active) seq_bounds(cu, s, total_len, max_seqlen, st, len);
    const int r0 = t * 64;
    const int i = r0 + l;
    const bool valid = active && i < len;
    int lo = 0x7fffffff, wcl = 0;
    if (valid) {
        const int wi = max(w[st + i], 1);
        lo = max(i - wi + 1, 0);
        wcl = min(wi, len);
    }
    const uint32_t khi = (uint32_t)lo >> 26, klo = ((uint32_t)lo << 6) | (uint32_t)l;  // key lo * 64 + l
    int rank = 0;
    for (int j = 0; j < 64; ++j) {
        const uint32_t jhi = (uint32_t)__builtin_amdgcn_readlane((int)khi, j);
        const uint32_t jlo = (uint32_t)__builtin_amdgcn_readlane((int)klo, j);
        rank += (jhi < khi || (jhi == khi && jlo < klo)) ? 1 : 0;
    }
    sp[rank] = l;
    slo[l] = lo;
    __syncthreads();
    const int pl = sp[l];  // row offset at sorted position l
    const int ri = r0 + pl;
    const bool rv = active && ri < len;
    int rlo = 0x7fffffff, rlmax = (int)0x80000000, rhi = -1, rhmin = 0x7fffffff;
    if (rv) {
        rlo = slo[pl];
        rlmax = rlo;
        rhi = ri;
        rhmin = ri;
    }
    rlo = row_min16(rlo);
    rlmax = row_max16(rlmax);
    rhi = row_max16(rhi);
    rhmin = row_min16(rhmin);
    const int m = row_max16(wcl);
    const int tm = max(max(__builtin_amdgcn_readlane(m, 0), __builtin_amdgcn_readlane(m, 16)),
                       max(__builtin_amdgcn_readlane(m, 32), __builtin_amdgcn_readlane(m, 48)));
    if (!active) return;
    o.perm[(int64_t)tile * 64 + l] = (uint8_t)pl;
    if ((l & 15) == 0) {
        int* b = o.bounds + ((int64_t)tile * 4 + (l >> 4)) * 4;
        b[0] = rlo;
        b[1] = rlmax;
        b[2] = rhi;
        b[3] = rhmin;
    }
    if (l == 0) o.wmax[tile] = tm;
}

}  // namespace dsalt

// mfma_map.h — the index and copy-address arithmetic of the staged MFMA
// kernels (mfma_sa_kernel, mfma_dma_kernel), as plain functions that compile
// for the device and for the host. The kernels call them; a host-side checker
// built from this same header walks every workgroup, wave, lane and block of
// a dispatch and asserts that each copy reads inside its buffer and that the
// workgroup -> work-item maps cover every item exactly once.
//
// Everything here is integer arithmetic on offsets (bytes unless a name says
// floats); no pointer is formed, so the host checker needs no buffers.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MMAP_HD __host__ __device__ __forceinline__
#else
#define MMAP_HD static inline
#endif

namespace phip {
namespace mmap {

constexpr int TILE_O = 32;    // rows of a weight tile in the device layout
constexpr int BLK = 32;       // K elements per block (one MFMA K step)
constexpr int MT_ROWS = 32;   // rows of one M tile

MMAP_HD int imin(int a, int b) { return a < b ? a : b; }

// ---- workgroup -> work item ------------------------------------------------

// Channel slabs of one projection: gate/up workgroups cover 4 x 32 channels
// of gate and of up (span = O rounded to 32), down workgroups 4 x 64.
MMAP_HD int slab_channels(bool gateup) { return gateup ? 4 * 32 : 4 * 32 * 2; }
MMAP_HD int slab_count(bool gateup, int O) {
    const int span = gateup ? ((O + 31) & ~31) : O;
    return (span + slab_channels(gateup) - 1) / slab_channels(gateup);
}

// XCD-aware order over n = NS * T items. The hardware deals workgroup L to
// XCD L mod 8; XCD x takes the contiguous run of items
// [x*q + min(x, r), ...) of length q + (x < r), with q = n / 8, r = n mod 8.
// For L < n this is a bijection onto [0, n) for every n; L >= n idles (-1).
MMAP_HD int xo_item(int L, int n) {
    if (L < 0 || L >= n) return -1;
    const int q = n >> 3, r = n & 7, x = L & 7, seq = L >> 3;
    return x * q + imin(x, r) + seq;
}

// Item -> (slab, tile) inside its expert, whose M tiles are [ts, ts + nt):
// the expert owns items [NS*ts, NS*(ts+nt)), ordered (group of G tiles, slab,
// tile in group), so the tiles of a group read each weight slab back to back.
constexpr int XO_G = 8;
MMAP_HD void xo_place(int item, int NS, int ts, int nt, int *slab, int *tile) {
    const int local = item - NS * ts;
    const int grp = local / (NS * XO_G), within = local - grp * NS * XO_G;
    const int gsize = imin(XO_G, nt - grp * XO_G);
    *slab = within / gsize;
    *tile = ts + grp * XO_G + (within - *slab * gsize);
}

// ---- copy sources ----------------------------------------------------------

// The activation dword a lane copies each block: row 8*wave + lane/8 of the
// tile (rows past the expert's end repeat its last row, never stored),
// column byte 4*(lane%8) of the 32-byte block.
MMAP_HD int a_row(int r0, int rend, int wave, int lane) {
    const int ra = r0 + 8 * wave + (lane >> 3);
    return ra < rend ? ra : rend - 1;
}
MMAP_HD uint32_t a_col(int lane) { return (uint32_t)(lane & 7) * 4; }

// Bytes of one 32-column subtile of one block, and of one 32-row weight tile.
MMAP_HD uint32_t sub_bytes(bool w4) { return 32u * (w4 ? 16u : 32u); }
MMAP_HD uint32_t tile_bytes(bool w4, int nb) { return (uint32_t)nb * sub_bytes(w4); }
MMAP_HD uint32_t stile_bytes(int ng) { return (uint32_t)ng * 128u; }   // one tile's scales

// mfma_sa_kernel: each wave copies two subtiles of one tensor (2w, 2w+1 of
// the stage). mat: 0 gate, 1 up, 2 down. Tiles past the tensor clamp to its
// last tile (never stored).
MMAP_HD int sa_mat(bool gateup, int wave) { return gateup ? (wave >> 1) : 2; }
MMAP_HD int sa_wtile(bool gateup, int slab, int wave, int q, int ntile) {
    const int t = gateup ? slab * 4 + 2 * (wave & 1) + q : slab * 8 + 2 * wave + q;
    return t < ntile ? t : ntile - 1;
}
// int4: lane half q = lane/32 copies subtile q, 16 bytes of column lane%32;
// per block the source advances by sub_bytes.
MMAP_HD uint32_t sa_voff_w4(bool gateup, int slab, int wave, int lane, int ntile, int nb) {
    return (uint32_t)sa_wtile(gateup, slab, wave, lane >> 5, ntile) * tile_bytes(true, nb) + (uint32_t)(lane & 31) * 16;
}
// int8: one copy per subtile q: lane covers half (lane%2) of column lane/2;
// the copy of subtile q adds sa_tile8(q).
MMAP_HD uint32_t sa_voff_w8(int lane) { return (uint32_t)(lane >> 1) * 32 + (uint32_t)(lane & 1) * 16; }
MMAP_HD uint32_t sa_tile8(bool gateup, int slab, int wave, int q, int ntile, int nb) {
    return (uint32_t)sa_wtile(gateup, slab, wave, q, ntile) * tile_bytes(false, nb);
}
// scales: one f32 of column lane%32 of subtile lane/32, per weight group.
MMAP_HD uint32_t sa_voff_s(bool gateup, int slab, int wave, int lane, int ntile, int ng) {
    return (uint32_t)sa_wtile(gateup, slab, wave, lane >> 5, ntile) * stile_bytes(ng) + (uint32_t)(lane & 31) * 4;
}

// mfma_dma_kernel: lane half sl = lane/32 covers channel group sl (gate/up:
// gate or up of this wave's 32 channels; down: the wave's two 32-channel
// subtiles). Channels past Op clamp to the last one (never stored).
MMAP_HD int dma_n0(bool gateup, int slab, int wave) {
    return gateup ? (slab * 4 + wave) * 32 : (slab * 4 + wave) * 64;
}
MMAP_HD int dma_ch(bool gateup, int n0, int lane, int Op) {
    const int o = gateup ? n0 + (lane & 31) : n0 + (lane >> 5) * 32 + (lane & 31);
    return o < Op ? o : Op - 1;
}
MMAP_HD int dma_mat(bool gateup, int lane) { return gateup ? (lane >> 5) : 2; }
// weight bytes of channel o at block 0 (int4: 16 bytes of that channel)
MMAP_HD uint32_t dma_w4(int o, int nb) {
    return ((uint32_t)(o / TILE_O) * (uint32_t)nb * TILE_O + (uint32_t)(o % TILE_O)) * 16u;
}
// int8, copy q: channel n0 + 32q (down) or n0 (gate/up, tensor q) + lane/2,
// 16-byte half lane%2 of its 32 bytes
MMAP_HD int dma_ch8(bool gateup, int n0, int lane, int q, int Op) {
    const int o = gateup ? n0 + (lane >> 1) : n0 + q * 32 + (lane >> 1);
    return o < Op ? o : Op - 1;
}
MMAP_HD uint32_t dma_w8(int o, int nb, int lane) {
    return ((uint32_t)(o / TILE_O) * (uint32_t)nb * TILE_O + (uint32_t)(o % TILE_O)) * 32u + (uint32_t)(lane & 1) * 16u;
}
// scales of channel o, in floats, at group 0 (a group advances by TILE_O)
MMAP_HD uint32_t dma_s(int o, int ng) { return (uint32_t)(o / TILE_O) * (uint32_t)ng * TILE_O + (uint32_t)(o % TILE_O); }

// Per-32 activation scales of the tile, copied once: copy i of a wave covers
// blocks 2i and 2i+1 (lane/32), row lane%32 (clamped like a_row).
MMAP_HD int sx_row(int r0, int rend, int lane) {
    const int rx = r0 + (lane & 31);
    return rx < rend ? rx : rend - 1;
}
MMAP_HD int sx_blk(int i, int lane, int nb) { return imin(2 * i + (lane >> 5), nb - 1); }

// Weight group of block b (per-row weights: gshift 30, every block in group 0).
MMAP_HD int grp_of_blk(int b, int gshift) { return gshift >= 30 ? 0 : b >> gshift; }

}  // namespace mmap
}  // namespace phip

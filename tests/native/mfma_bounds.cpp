// Host-side bounds checker for the staged MFMA kernels' copies.
//
// It walks every workgroup of one dispatch exactly as mfma_sa_kernel and
// mfma_dma_kernel map it (the same functions, from
// peregrine_amd/csrc/mfma_map.h), and for every wave, lane and K block checks
// that each LDS-DMA copy reads inside its buffer:
//   activations  xq  [rows_x][x_stride] int8   (4 bytes per lane per block)
//   weights      w   [Op/32][nb][32][BB]       (16 bytes per lane per copy)
//   scales       sc  [Op/32][ng][32] f32       (4 bytes per lane per block)
//   act. scales  sx  [rows_x][sx_stride] f32   (per-32 mode, preloaded once)
// and that the workgroups cover every (M tile, channel slab) item exactly
// once. Returns the number of violations; the first few are printed.
#include <cstdio>
#include <vector>

#include "../../peregrine_amd/csrc/mfma_map.h"

using namespace phip::mmap;

struct Geom {
    int K, Kp, nb, O, Op, ng, gshift, w4;
};

static long g_bad = 0;
static void bad(const char *what, long a, long b, long c, long d) {
    if (g_bad++ < 8) std::fprintf(stderr, "mfma_bounds: %s (%ld %ld %ld %ld)\n", what, a, b, c, d);
}

static void need(bool ok, const char *what, long a, long b, long c, long d) {
    if (!ok) bad(what, a, b, c, d);
}

// kind: 0 = mfma_sa_kernel, 1 = mfma_dma_kernel. xo: the XCD-aware order
// (sa kernel, weight-reuse dispatches). b32: per-32 activation scales (the
// scale preload and the per-block weight-scale copies); grp_copy: the
// per-block weight-scale copy runs (every epilogue but per-row weights).
extern "C" long check_dispatch(int kind, int gateup, int xo, int b32, int grp_copy, const Geom *g, int T,
                               int grid_tiles, const int *mt_exp, const int *mt_row0, const int *mt_rend,
                               const int *mt_first, int R, const int *row_act, int rows_x, int x_stride,
                               int sx_stride, int n_desc) {
    g_bad = 0;
    const int NS = slab_count(gateup != 0, g->O);
    const int ntile = g->Op / TILE_O;
    const long w_bytes = (long)g->Op * g->nb * (g->w4 ? 16 : 32);
    const long s_bytes = (long)g->Op * g->ng * 4;
    const long x_bytes = (long)rows_x * x_stride;
    const long sx_floats = (long)rows_x * sx_stride;
    need(g->Kp <= x_stride, "x_stride below Kp", g->Kp, x_stride, 0, 0);
    need(!b32 || g->nb <= sx_stride, "sx_stride below nb", g->nb, sx_stride, 0, 0);
    std::vector<int> seen((size_t)NS * (T > 0 ? T : 1), 0);
    for (int by = 0; by < grid_tiles; ++by) {
        for (int bx = 0; bx < NS; ++bx) {
            int tile = by, slab = bx;
            if (xo) {
                const int item = xo_item(bx + NS * by, NS * T);
                if (item < 0) continue;
                const int q = item / NS;
                need(q >= 0 && q < T, "xo item tile", item, q, T, 0);
                const int ts = mt_first[q];
                const int nt = (mt_rend[q] - mt_row0[ts] + MT_ROWS - 1) / MT_ROWS;
                xo_place(item, NS, ts, nt, &slab, &tile);
                need(slab >= 0 && slab < NS && tile >= ts && tile < ts + nt, "xo place", item, slab, tile, ts);
                if (!(slab >= 0 && slab < NS && tile >= 0 && tile < T)) continue;
            }
            if (tile >= T) continue;
            seen[(size_t)tile * NS + slab]++;
            const int e = mt_exp[tile], r0 = mt_row0[tile], rend = mt_rend[tile];
            need(e >= 0 && e < n_desc, "descriptor index", tile, e, n_desc, 0);
            need(r0 >= 0 && r0 < rend && rend <= R, "tile rows", tile, r0, rend, R);
            if (!(r0 >= 0 && r0 < rend && rend <= R)) continue;
            auto act = [&](int r) { return row_act ? row_act[r] : r; };
            for (int wave = 0; wave < 4; ++wave) {
                for (int lane = 0; lane < 64; ++lane) {
                    const int ra = a_row(r0, rend, wave, lane);
                    const int xr = act(ra);
                    need(xr >= 0 && xr < rows_x, "activation row", tile, ra, xr, rows_x);
                    const long a0 = (long)xr * x_stride + a_col(lane);
                    long w0[2] = {0, 0}, s0;
                    int nw = 1;
                    if (kind == 0) {
                        if (g->w4) {
                            w0[0] = sa_voff_w4(gateup != 0, slab, wave, lane, ntile, g->nb);
                        } else {
                            nw = 2;
                            for (int q = 0; q < 2; ++q)
                                w0[q] = (long)sa_voff_w8(lane) + sa_tile8(gateup != 0, slab, wave, q, ntile, g->nb);
                        }
                        s0 = sa_voff_s(gateup != 0, slab, wave, lane, ntile, g->ng);
                    } else {
                        const int n0 = dma_n0(gateup != 0, slab, wave);
                        const int o = dma_ch(gateup != 0, n0, lane, g->Op);
                        if (g->w4) {
                            w0[0] = dma_w4(o, g->nb);
                        } else {
                            nw = 2;
                            for (int q = 0; q < 2; ++q) w0[q] = dma_w8(dma_ch8(gateup != 0, n0, lane, q, g->Op), g->nb, lane);
                        }
                        s0 = (long)dma_s(o, g->ng) * 4;
                    }
                    const long wstep = g->w4 ? 16L * 32 : 32L * 32;   // one block of a 32-row tile
                    for (int b = 0; b < g->nb; ++b) {
                        const long ab = a0 + (long)b * BLK;
                        need(ab >= 0 && ab + 4 <= x_bytes && (long)b * BLK + a_col(lane) + 4 <= g->Kp,
                             "activation copy", tile, wave, lane, b);
                        for (int q = 0; q < nw; ++q) {
                            const long wb = w0[q] + (long)b * wstep;
                            need(wb >= 0 && wb + 16 <= w_bytes, "weight copy", tile, slab, wave * 64 + lane, b);
                        }
                        if (grp_copy) {
                            const int gi = grp_of_blk(b, g->gshift);
                            const long sb = s0 + (long)gi * (kind == 0 ? 128 : TILE_O * 4);
                            need(gi < g->ng && sb >= 0 && sb + 4 <= s_bytes, "scale copy", tile, slab, wave * 64 + lane, b);
                        }
                    }
                    if (b32) {
                        const int rx = act(sx_row(r0, rend, lane));
                        for (int i = wave; i < (g->nb + 1) >> 1; i += 4) {
                            const long f = (long)rx * sx_stride + sx_blk(i, lane, g->nb);
                            need(rx >= 0 && rx < rows_x && f >= 0 && f < sx_floats, "act scale copy", tile, rx, i, lane);
                        }
                    }
                }
            }
        }
    }
    for (int t = 0; t < T; ++t)
        for (int s = 0; s < NS; ++s) need(seen[(size_t)t * NS + s] == 1, "item coverage", t, s, seen[(size_t)t * NS + s], NS);
    return g_bad;
}

extern "C" int xo_item_c(int L, int n) { return xo_item(L, n); }

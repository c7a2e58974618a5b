// Host-side check of the f32 prefill's stream-K partition (skgeo.h), built
// with g++ by tests/test_skgeo.py. For each shape it walks every workgroup's
// unit range exactly as k_fa_f32 does and checks that: the ranges are
// non-empty and cover every unit once; a block covered whole is written by
// one workgroup; a cut block's partials sit in distinct slots, which the
// merge's arithmetic (wg_at, lo) finds again, in workgroup order; no
// workgroup cuts more than its first and last block; and the XCD numbering of
// the workgroups (xcd_order) is a bijection. Prints "ok <shapes>" or
// the first failure. It also checks floordiv_nn, the division these walks
// and the decode attention's partition use, against the integer quotient.
#define __host__
#define __device__
#include <cstdio>
#include <cstdlib>
#include <map>
#include <set>
#include <vector>

#include "skgeo.h"

using tn::SkGeo;

static int check(int64_t BH, int L, int S, int causal, int BQ, int BK, int slots) {
    SkGeo geo;
    geo.nqb = (L + BQ - 1) / BQ;
    geo.NS = (S + BK - 1) / BK;
    geo.c = BQ / BK;
    geo.causal = causal;
    geo.Tbh = geo.P(geo.nqb);
    geo.T = BH * geo.Tbh;
    geo.G = slots < geo.T ? slots : geo.T;
    if (geo.G < 1) geo.G = 1;
    // the walk of k_fa_f32: (block id) -> list of (workgroup, slot) for cut blocks
    std::map<int64_t, std::vector<std::pair<int64_t, int64_t>>> parts;
    std::map<int64_t, int> whole;
    std::vector<int> seen(geo.T, 0);
    if (geo.lo(0) != 0 || geo.lo(geo.G) != geo.T) return 1;
    {
        // xcd_order is a bijection of 0 .. G-1, and the workgroups one XCD
        // takes (b = x, x + 8, ...) get consecutive range numbers
        std::vector<int> hit(geo.G, 0);
        for (int64_t b = 0; b < geo.G; b++) {
            const int64_t g = geo.xcd_order(b);
            if (g < 0 || g >= geo.G || hit[g]++) return 12;
            if (b >= 8 && g != geo.xcd_order(b - 8) + 1) return 13;
        }
    }
    for (int64_t g = 0; g < geo.G; g++) {
        const int64_t u_lo = geo.lo(g), u_hi = geo.lo(g + 1);
        if (u_hi <= u_lo) return 2;  // an empty range
        int64_t u = u_lo;
        bool first = true;
        int cuts = 0;
        while (u < u_hi) {
            int64_t bh;
            int qt, t0;
            geo.locate(u, bh, qt, t0);
            const int n = geo.nt(qt);
            const int t1 = (int)(t0 + (u_hi - u) < n ? t0 + (u_hi - u) : n);
            for (int64_t x = u; x < u + (t1 - t0); x++) {
                seen[x]++;
                if (geo.wg_of(x) != g) return 3;  // the inverse disagrees with lo
            }
            const int64_t blk = bh * geo.nqb + qt;
            if (t0 == 0 && t1 == n) {
                whole[blk]++;
            } else {
                parts[blk].push_back({g, 2 * g + (first ? 0 : 1)});
                if (!first && u + (t1 - t0) != u_hi) return 4;  // a later cut block must end the range
                cuts++;
            }
            u += t1 - t0;
            first = false;
        }
        if (cuts > 2) return 5;
    }
    for (int64_t x = 0; x < geo.T; x++)
        if (seen[x] != 1) return 6;
    for (auto& kv : whole)
        if (kv.second != 1 || parts.count(kv.first)) return 7;
    std::set<int64_t> slots_used;
    for (auto& kv : parts) {
        const int64_t bh = kv.first / geo.nqb;
        const int qt = (int)(kv.first % geo.nqb);
        const int n = geo.nt(qt);
        const int64_t u0 = bh * geo.Tbh + geo.P(qt);
        // the merge's arithmetic in k_fa_f32
        const int64_t g_lo = geo.wg_of(u0), g_hi = geo.wg_of(u0 + n - 1);
        const int64_t s_lo = 2 * g_lo + (geo.lo(g_lo) < u0 ? 1 : 0);
        const auto& v = kv.second;
        if ((int64_t)v.size() != g_hi - g_lo + 1) return 8;
        for (size_t i = 0; i < v.size(); i++) {
            const int64_t want_g = g_lo + (int64_t)i;
            const int64_t want_s = i == 0 ? s_lo : 2 * want_g;
            if (v[i].first != want_g || v[i].second != want_s) return 9;
            if (!slots_used.insert(v[i].second).second) return 10;
            if (v[i].second >= 2 * geo.G) return 11;
        }
    }
    return 0;
}

// floordiv_nn against the integer quotient: near multiples of t (where the
// f64 quotient rounds to the next integer), at the ends of the range the
// kernels use (products below 2^42), and on a pseudo-random sweep
static int check_div() {
    const int64_t ts[] = {1, 2, 3, 7, 255, 256, 1023, 1024, 2047, 2048, 65535, 1000003, 2147483647LL};
    for (int64_t t : ts)
        for (int64_t k : {0LL, 1LL, 2LL, 1000LL, (1LL << 20) + 7, (1LL << 31) - 1, (1LL << 42) / t})
            for (int64_t d = -2; d <= 2; d++) {
                const int64_t x = k * t + d;
                if (x < 0) continue;
                if (tn::floordiv_nn(x, t) != x / t) return 1;
            }
    uint64_t r = 0x9e3779b97f4a7c15ULL;
    for (int i = 0; i < 2000000; i++) {
        r ^= r << 13;
        r ^= r >> 7;
        r ^= r << 17;
        const int64_t x = (int64_t)(r >> 22), t = (int64_t)((r & 0x7fffffff) | 1) >> (r % 31);
        if (t < 1) continue;
        if (tn::floordiv_nn(x, t) != x / t) return 1;
    }
    return 0;
}

int main() {
    int n = 0;
    if (check_div()) {
        std::printf("fail: floordiv_nn\n");
        return 1;
    }
    const int Ls[] = {1, 5, 127, 128, 129, 300, 1000, 2048, 4096};
    const int Ss[] = {1, 63, 64, 65, 200, 1000, 2048, 4096};
    const int64_t BHs[] = {1, 2, 9, 32, 64};
    const int slotss[] = {1, 7, 64, 255, 512, 1024};
    for (int64_t BH : BHs)
        for (int L : Ls)
            for (int S : Ss)
                for (int causal = 0; causal < 2; causal++)
                    for (int bk : {64, 32})
                        for (int slots : slotss) {
                            if (BH * (int64_t)L * S > (int64_t)64 * 4096 * 4096 / 4) continue;
                            const int r = check(BH, L, S, causal, 128, bk, slots);
                            if (r) {
                                std::printf("fail %d: BH=%lld L=%d S=%d causal=%d bk=%d slots=%d\n", r, (long long)BH, L,
                                            S, causal, bk, slots);
                                return 1;
                            }
                            n++;
                        }
    std::printf("ok %d\n", n);
    return 0;
}

// Stream-K partition of the f32 prefill (k_fa_f32 in sdpa.hip).
//
// A unit is one key tile of one PF_BQ-query block; units run over (batch *
// head, query block, key tile) in that order, a query block qt having nt(qt)
// key tiles. The persistent grid's G workgroups take equal unit ranges
// [g T / G, (g+1) T / G), so every workgroup does the same MFMA work whatever
// the causal shape. A workgroup writes a query block it covers whole straight
// to the output; a block cut by a range boundary leaves an unnormalised
// (O, m, l) partial per workgroup: in slot 2g if it is workgroup g's first
// block, else 2g + 1 (a workgroup cuts at most its first and its last block),
// and the workgroup that finishes the block last merges them in workgroup
// order.
//
// The host and device compilers both read this header; a host-only build
// defines __host__ and __device__ before including it.
#pragma once
#include <cstdint>

namespace tn {

// floor(x / t) for 0 <= x < 2^53 and t > 0: the quotient from f64 (exact
// operands, so it is off by at most one) corrected in integers. On the GPU a
// 64-bit integer division is a long instruction sequence; this is a few.
__host__ __device__ inline int64_t floordiv_nn(int64_t x, int64_t t) {
    int64_t q = (int64_t)((double)x / (double)t);
    if (q * t > x) q--;
    else if ((q + 1) * t <= x) q++;
    return q;
}

struct SkGeo {
    int nqb, NS, c, causal;  // query blocks, key tiles of S, key tiles per query block (PF_BQ / BK)
    int64_t Tbh, T, G;       // units per (batch, head), all units, workgroups (G <= T)
    __host__ __device__ int nt(int qt) const { return causal ? (c * (qt + 1) < NS ? c * (qt + 1) : NS) : NS; }
    // units of query blocks 0 .. qt-1 of one (batch, head)
    __host__ __device__ int64_t P(int qt) const {
        if (!causal) return (int64_t)qt * NS;
        const int64_t m = qt < NS / c ? qt : NS / c;  // blocks below qt whose tiles stop before S
        return (int64_t)c * m * (m + 1) / 2 + ((int64_t)qt - m) * NS;
    }
    __host__ __device__ int64_t lo(int64_t g) const { return floordiv_nn(g * T, G); }
    // The range number of hardware workgroup b. Workgroups are dealt to the
    // eight XCDs in turn (b to XCD b % 8); XCD x takes the consecutive
    // numbers x*(G/8) + min(x, G%8) onwards, so that the ranges of one head
    // stay on one or two XCDs' L2s. A bijection of 0 .. G-1.
    __host__ __device__ int64_t xcd_order(int64_t b) const {
        const int64_t x = b % 8, qx = G / 8, rx = G % 8;
        return x * qx + (x < rx ? x : rx) + b / 8;
    }
    // ceil((u + 1) G / T) - 1
    __host__ __device__ int64_t wg_of(int64_t u) const { return floordiv_nn((u + 1) * G - 1, T); }
    // the query block (bh, qt) that holds unit u, and u's tile in it
    __host__ __device__ void locate(int64_t u, int64_t& bh, int& qt, int& t) const {
        bh = floordiv_nn(u, Tbh);
        const int64_t r = u - bh * Tbh;
        int a = 0, b = nqb;  // the largest qt with P(qt) <= r (every block has a tile)
        while (b - a > 1) {
            const int mid = (a + b) >> 1;
            if (P(mid) <= r) a = mid; else b = mid;
        }
        qt = a;
        t = (int)(r - P(a));
    }
};

}  // namespace tn

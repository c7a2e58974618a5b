// bf16 / f16 SDPA prefill at head dim 64 without split rows.
//
// Same semantics as the other prefill kernels (sdpa.hip; the reference's
// aten._scaled_dot_product_flash_attention_for_cpu, aten.rs:10092-10440):
// softmax(q k^T * scale [+ mask] [+ upper-left causal -inf]) v with f32
// accumulation, the probabilities narrowed to the input format between the
// two products (flash.rs:503-516), GQA by indexing key/value head
// h / (Hq/Hkv), lse over the masked, scaled scores.
//
// Shape of the work. One workgroup owns a 64-query block of one (batch,
// head) and the whole of its key range, so no row is split across
// workgroups and nothing is merged through memory; with causal rows the
// workgroups are issued longest first. Its sixteen waves are two query
// halves of 32 times eight key groups: a 256-key ring stage holds eight
// 32-key tiles, and tile g of every stage is computed by waves 2g (queries
// 0-31) and 2g + 1 (queries 32-63), so every K/V byte brought into LDS serves
// 64 queries. The key groups meet in LDS once, at the end.
//
// Why sixteen waves. On gfx950 one wave issues VALU instructions at about
// half the rate a SIMD can execute them (measured: 7.6 cycles per wave64
// FMA for one wave, 8.6 each for two waves sharing a SIMD), and the softmax
// is VALU-bound, so a SIMD needs two waves in their softmax at once to be
// busy, while others feed the matrix core. Four waves per SIMD (128 VGPRs
// each) give that without any explicit scheduling: the waves of a stage
// start together, their score products queue on the matrix core, and they
// leave for their softmax one after another.
//
// Per tile and wave (as k_flash16 in sdpa.hip): S^T = K . Q^T on
// v_mfma_f32_32x32x16 with Q^T in registers (read once from the block's
// query rows, staged in LDS by one load per 16-byte chunk) and K rows from the
// XOR-swizzled ring, lane l owning query l & 31; P = exp2(S*scale*log2e - m)
// narrowed RNE; O^T += V^T . P^T with V^T read column-wise by
// ds_read_b64_tr_b16. The reference point m of a row moves only when it
// must: a row's first tile sets it to that tile's maximum before any
// exponential; after that the probabilities are computed against the
// current m, and only if a lane's sum of its sixteen probabilities exceeds
// 2^10 (so no probability is larger) is the tile's maximum taken, m moved to
// it, the accumulators rescaled and the probabilities recomputed. That is
// the same softmax, and it drops the row maximum from the common path.
#include "tn_common.h"
#include "attn_common.h"

namespace tn {
namespace {

constexpr int FA_D = 64;
constexpr int FA_BQ = 64;                 // queries per workgroup: two halves of 32
constexpr int FA_KG = 8;                  // key groups
constexpr int FA_BKW = 32;                // keys per tile
constexpr int FA_ROWS = FA_KG * FA_BKW;   // keys per ring stage
constexpr int FA_NT = 1024;               // sixteen waves
constexpr float FA_SUM_MAX = 1024.0f;     // a lane's probability sum that moves the reference point

template <int MASK, bool F16>
__global__ __launch_bounds__(FA_NT) void k_fa64(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kg,
                                                const uint16_t* __restrict__ Vg, int BH, int Hq, int Hkv, int L,
                                                int S, int nqb, float sl2, int causal, uint16_t* __restrict__ Og,
                                                float* __restrict__ lse, const MaskRef mask) {
    constexpr int D = FA_D;
    constexpr int CPR = D / 8;                         // 16-byte chunks per row
    constexpr int STAGE = FA_ROWS * D;                 // elements of one K (or V) stage
    constexpr int LPT = FA_ROWS * CPR / FA_NT;         // 16-byte loads per thread per stage, K and V each
    constexpr int NW = FA_NT / 64;
    static_assert(LPT * FA_NT == FA_ROWS * CPR, "stage must split evenly over the threads");
    // one LDS object per ring stage: with the stage known at compile time
    // the compiler can tell a read of one stage from the loads landing in the
    // other and emits no blanket vmcnt(0) in front of it
    __shared__ __align__(16) uint16_t sK0[STAGE], sK1[STAGE];
    __shared__ __align__(16) uint16_t sV0[STAGE], sV1[STAGE];
    __shared__ float2 s_ml[NW][32];  // each wave's (m, l) per query row
    // a mask that is the same for every query row: the stage's 256 values,
    // in log2 units, per ring stage
    __shared__ __align__(16) float sM[MASK ? 2 : 1][MASK ? FA_ROWS : 1];
    __shared__ __align__(16) uint16_t sQ[FA_BQ * D];  // the block's query rows, chunks swizzled as K's
    auto stK = [&](auto sc) -> uint16_t* {
        if constexpr (decltype(sc)::value == 0) return sK0; else return sK1;
    };
    auto stV = [&](auto sc) -> uint16_t* {
        if constexpr (decltype(sc)::value == 0) return sV0; else return sV1;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qh = w & 1, kg = w >> 1;  // query half, key group
    const int lq = lane & 31, hh = lane >> 5;
    // longest rows first: with causal rows, query block nqb-1 of every (batch, head) comes first
    const int item = (int)blockIdx.x;
    const int qt = causal ? nqb - 1 - item / BH : item / BH;
    const int bh = item % BH;
    const int h = bh % Hq, b = bh / Hq;
    const int kvh = h / (Hq / Hkv);
    const int q0 = qt * FA_BQ;
    const int qw0 = q0 + 32 * qh;  // this wave's first query
    const int qi = qw0 + lq;
    const int kend = causal ? min(S, q0 + FA_BQ) : S;  // upper-left: row i sees keys 0..i
    const int nst = (kend + FA_ROWS - 1) / FA_ROWS;

    const uint16_t* qp = Qg + ((int64_t)b * Hq + h) * L * D;
    const uint16_t* kp = Kg + ((int64_t)b * Hkv + kvh) * S * D;
    const uint16_t* vp = Vg + ((int64_t)b * Hkv + kvh) * S * D;

    // physical 16-byte chunk of logical chunk c in row r (an involution)
    auto swz = [](int r, int c) { return c ^ ((r >> 1) & 7); };

    using E = El<F16>;
    using V8 = typename E::v8;
    // The block's 64 query rows come into LDS once (8 KB, rows past L read
    // as 0), one 1 KB LDS-DMA load for each of waves 0-7, ahead of the first
    // stage's K and V: each of the eight key groups of a query half needs
    // the same rows, and the CU's vector memory path takes a workgroup's
    // first loads one instruction after another.
    if (w < FA_BQ * CPR / 64) {
        const int p = 64 * w + lane;
        const int row = p / CPR;
        const buf_rsrc rq = make_rsrc(qp + (int64_t)q0 * D, (uint32_t)(L - q0) * (uint32_t)(D * 2));
        lds_direct16(rq, (uint32_t)(row * D + swz(row, p % CPR) * 8) * 2u, sQ + 64 * w * 8);
    }
    // Q^T operand: lane l holds q[qw0 + (l&31)][16c + 8*(l>>5) .. +7], read
    // from sQ after the first stage's barrier
    V8 qf[D / 16];

    // this lane's byte offset in a stage for its i-th 16-byte load (LDS chunk
    // position p = tid + NT*i holds logical chunk swz(row, p % CPR) of row p / CPR)
    uint32_t voff[LPT];
#pragma unroll
    for (int i = 0; i < LPT; i++) {
        const int p = tid + FA_NT * i;
        const int row = p / CPR;
        voff[i] = (uint32_t)(row * D + swz(row, p % CPR) * 8) * 2u;
    }
    // the mask row of this (batch, head); thread t < 256 loads key t of each
    // stage into mval, and writes it to sM once the stage's loads have landed
    const int64_t mbase = MASK ? (int64_t)b * mask.sb + (int64_t)h * mask.sh : 0;
    float mval = 0.0f;
    auto issue = [&](auto sc, int st) __attribute__((always_inline)) {
        const int k0 = st * FA_ROWS;
        if constexpr (MASK != 0) {
            const int key = k0 + tid;
            mval = 0.0f;  // keys past S: masked by the tile's key test
            if (tid < FA_ROWS && key < S) mval = mask_val<MASK, F16>(mask.p, mbase + (int64_t)key * mask.sk);
        }
        const uint32_t bytes = (uint32_t)(S - k0) * (uint32_t)(D * 2);  // keys k0 .. S-1; past them read 0
        const buf_rsrc rk = make_rsrc(kp + (int64_t)k0 * D, bytes);
        const buf_rsrc rv = make_rsrc(vp + (int64_t)k0 * D, bytes);
        uint16_t* dK = stK(sc);
        uint16_t* dV = stV(sc);
#pragma unroll
        for (int i = 0; i < LPT; i++) {
            lds_direct16(rk, voff[i], dK + (w + NW * i) * 64 * 8);
            lds_direct16(rv, voff[i], dV + (w + NW * i) * 64 * 8);
        }
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    const float scl = MASK ? 1.0f : sl2;  // scores' factor to log2 units
    const int gi = lane & 15;
    const int dcol = 16 * ((lane >> 4) & 1) + 4 * (gi & 3);  // V^T operand: source lane's 4 columns

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    issue(I0{}, 0);  // nst >= 1
    wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int c = 0; c < D / 16; c++) {
        const int row = 32 * qh + lq;
        qf[c] = *reinterpret_cast<const V8*>(sQ + row * D + swz(row, 2 * c + hh) * 8);
    }

    auto step = [&](auto sc, int st) __attribute__((always_inline)) {
        wait_vmcnt<0>();  // the only loads in flight are this stage's
        // the stage's mask values, in log2 units (the buffer's last reads,
        // two stages back, are behind the previous barrier)
        if constexpr (MASK != 0)
            if (tid < FA_ROWS) sM[decltype(sc)::value][tid] = mval * LOG2E;
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (st + 1 < nst) issue(std::integral_constant<int, 1 - decltype(sc)::value>{}, st + 1);

        const int k0 = st * FA_ROWS + FA_BKW * kg;
        // past the keys, or (causal) every query of the wave precedes the tile
        if (k0 >= kend || (causal && k0 > qw0 + 31)) return;
        const uint16_t* tK = stK(sc);
        const uint16_t* tV = stV(sc);
        const int kr = FA_BKW * kg;
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0.0f;
        // the tile's K fragments all read before the products: interleaved
        // with them by the compiler, two reads at a time, the LDS latency was
        // exposed twice per tile (the same for V below)
        V8 ka[D / 16];
#pragma unroll
        for (int c = 0; c < D / 16; c++) {
            const int row = kr + lq;
            ka[c] = *reinterpret_cast<const V8*>(tK + row * D + swz(row, 2 * c + hh) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < D / 16; c++) acc = E::mfma(ka[c], qf[c], acc);
        // The scores are read by VALU next. A VALU read of a 16-pass XDL
        // result needs 18 wait states; they are spelled out, tied to the
        // accumulator, so that no read is scheduled above them (the
        // compiler's hazard pass has missed them behind a branch).
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(acc));
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = acc[r];
        if constexpr (MASK != 0) {
            // scores to log2 units with the mask added, one rounding:
            // fma(raw, scale*log2e, mask*log2e)
            const float* ms = sM[decltype(sc)::value] + kr + 4 * hh;
#pragma unroll
            for (int rq = 0; rq < 4; rq++) {
                const float4 mv = *reinterpret_cast<const float4*>(ms + 8 * rq);
                v[4 * rq] = __builtin_fmaf(v[4 * rq], sl2, mv.x);
                v[4 * rq + 1] = __builtin_fmaf(v[4 * rq + 1], sl2, mv.y);
                v[4 * rq + 2] = __builtin_fmaf(v[4 * rq + 2], sl2, mv.z);
                v[4 * rq + 3] = __builtin_fmaf(v[4 * rq + 3], sl2, mv.w);
            }
        }
        if (k0 + FA_BKW > S || (causal && k0 + FA_BKW - 1 > qw0)) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = k0 + 8 * (r >> 2) + 4 * hh + (r & 3);
                if (key >= S || (causal && key > qi)) v[r] = -INFINITY;
            }
        }
        // A row with no reference point yet (this key group's first tile of
        // it) takes the tile's maximum before any exponential, so that its
        // probabilities are computed once. Rows that have one keep it.
        if (__any(m == -INFINITY)) {
            float a = max3f(v[0], v[1], v[2]);
            a = max3f(a, v[3], v[4]);
            a = max3f(a, v[5], v[6]);
            float bm = max3f(v[8], v[9], v[10]);
            bm = max3f(bm, v[11], v[12]);
            bm = max3f(bm, v[13], v[14]);
            const float mx = xor32_max(max3f(max3f(a, v[7], v[15]), bm, bm)) * scl;
            // o and l are still 0 for such a row: nothing to rescale
            if (m == -INFINITY) m = mx;
        }
        // probabilities against the current reference point
        float p[16], ps = 0.0f;
        {
            const float mu = (m == -INFINITY) ? 0.0f : m;
#pragma unroll
            for (int r = 0; r < 16; r++) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[r], scl, -mu));
#pragma unroll
            for (int r = 0; r < 16; r += 4) ps = ps + ((p[r] + p[r + 1]) + (p[r + 2] + p[r + 3]));
        }
        // a probability may exceed 2^10 (or one overflowed): move the
        // reference to the tile's maximum
        if (__any(!(ps <= FA_SUM_MAX))) {
            float a = max3f(v[0], v[1], v[2]);
            a = max3f(a, v[3], v[4]);
            a = max3f(a, v[5], v[6]);
            float bm = max3f(v[8], v[9], v[10]);
            bm = max3f(bm, v[11], v[12]);
            bm = max3f(bm, v[13], v[14]);
            const float mx = xor32_max(max3f(max3f(a, v[7], v[15]), bm, bm)) * scl;
            const float mn = fmaxf(m, mx);
            // a row with no key seen yet keeps m = mn = -inf: alpha 1, not 2^NaN
            const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
            l = l * alpha;
#pragma unroll
            for (int i = 0; i < D / 32; i++) o[i] = o[i] * alpha;
            m = mn;
            const float mu = (m == -INFINITY) ? 0.0f : m;
            ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[r], scl, -mu));
#pragma unroll
            for (int r = 0; r < 16; r += 4) ps = ps + ((p[r] + p[r + 1]) + (p[r + 2] + p[r + 3]));
        }
        l = l + ps;
        V8 pf[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
            pf[j] = __builtin_bit_cast(
                V8, make_uint4(E::pack_p(p[8 * j], p[8 * j + 1]), E::pack_p(p[8 * j + 2], p[8 * j + 3]),
                               E::pack_p(p[8 * j + 4], p[8 * j + 5]), E::pack_p(p[8 * j + 6], p[8 * j + 7])));
        V8 vf[D / 32][2];
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int r0 = kr + 16 * j + 4 * hh + (gi >> 2);
                const int r1 = r0 + 8;
                const int col = 32 * dt + dcol;
                const uint2 lo = lds_read_tr16(tV + r0 * D + swz(r0, col >> 3) * 8 + (col & 7));
                const uint2 hi = lds_read_tr16(tV + r1 * D + swz(r1, col >> 3) * 8 + (col & 7));
                vf[dt][j] = __builtin_bit_cast(V8, make_uint4(lo.x, lo.y, hi.x, hi.y));
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int j = 0; j < 2; j++) o[dt] = E::mfma(vf[dt][j], pf[j], o[dt]);
    };
    // the ring unrolled so that every stage index is a constant
    for (int st = 0; st < nst; st += 2) {
        step(I0{}, st);
        if (st + 1 < nst) step(I1{}, st + 1);
    }
    // the accumulators are read by VALU and LDS stores below, past the loop's
    // exit branch: the XDL wait states, spelled out as for the scores
#pragma unroll
    for (int i = 0; i < D / 32; i++) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(o[i]));
    l = xor32_sum(l);

    // The eight key groups of each query half meet in LDS. Each wave writes
    // its unscaled accumulators (8 KB) into a slot laid over the ring, with
    // its (m, l) beside it; then every thread takes one query's largest
    // reference point mu over the key groups and adds four columns of that
    // query over the groups in key-group order, each group's columns and l
    // scaled by 2^(m - mu) as they are read, normalises and stores them.
    // During the last stage the ring buffer it does not use is free, so the
    // waves of key groups 0-3 (the oldest, which finish their last tile
    // first) write there at once; groups 4-7 write over the last stage's
    // buffer once every wave has passed the barrier after its last reads.
    // Rows hold 16 float4 columns, XOR-swizzled by the query so that the 32
    // queries of a store land in different banks.
    const int lastbuf = (nst - 1) & 1;  // the ring buffer of the last stage
    auto slot_of = [&](int wv) -> float* {
        const int buf = wv < 8 ? lastbuf ^ 1 : lastbuf, a = (wv >> 2) & 1;
        uint16_t* base = buf == 0 ? (a == 0 ? sK0 : sV0) : (a == 0 ? sK1 : sV1);
        return reinterpret_cast<float*>(base) + (wv & 3) * (32 * D);
    };
    auto store_o = [&]() __attribute__((always_inline)) {
        float* slot = slot_of(w);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                // O^T[d = 32dt + 8g4 + 4hh + e][q = lq]
                const int c4 = (32 * dt + 8 * g4 + 4 * hh) >> 2;
                *reinterpret_cast<float4*>(slot + lq * D + ((c4 ^ (lq & 15)) << 2)) =
                    make_float4(o[dt][4 * g4], o[dt][4 * g4 + 1], o[dt][4 * g4 + 2], o[dt][4 * g4 + 3]);
            }
    };
    if (hh == 0) s_ml[w][lq] = make_float2(m, l);
    if (kg < 4) store_o();
    __syncthreads();
    if (kg >= 4) store_o();
    __syncthreads();
    {
        const int q = tid >> 4, c4 = tid & 15;  // query of the workgroup, columns 4*c4 .. 4*c4 + 3
        const int half = q >> 5, ql = q & 31;
        const int qrow = q0 + q;
        if (qrow < L) {
            float2 mlg[FA_KG];
            float mm = -INFINITY;
#pragma unroll
            for (int g = 0; g < FA_KG; g++) {
                mlg[g] = s_ml[2 * g + half][ql];
                mm = fmaxf(mm, mlg[g].x);
            }
            const float mu = (mm == -INFINITY) ? 0.0f : mm;
            float tl = 0.0f, a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
            for (int g = 0; g < FA_KG; g++) {
                // a group that saw no key has m = -inf: factor 0 (its o and l are 0)
                const float f = __builtin_amdgcn_exp2f(mlg[g].x - mu);
                tl = tl + mlg[g].y * f;
                const float4 x = *reinterpret_cast<const float4*>(slot_of(2 * g + half) + ql * D +
                                                                  ((c4 ^ (ql & 15)) << 2));
                a0 = a0 + x.x * f;
                a1 = a1 + x.y * f;
                a2 = a2 + x.z * f;
                a3 = a3 + x.w * f;
            }
            // the reciprocal (1 ulp) then four products: the bf16/f16 outputs
            // round far coarser than the f32 quotient's last bit
            const float inv = __builtin_amdgcn_rcpf(tl);
            const int64_t row = (int64_t)bh * L + qrow;
            *reinterpret_cast<uint2*>(Og + row * D + 4 * c4) =
                make_uint2(E::pack_out_hw(a0 * inv, a1 * inv), E::pack_out_hw(a2 * inv, a3 * inv));
            if (lse && c4 == 0) lse[row] = mm == -INFINITY ? NAN : mm * LN2 + logf(tl);
        }
    }
}

}  // namespace

// Launch for bf16 / f16 at head dim 64 (scale >= 0: the row maximum is
// taken over the unscaled scores). One workgroup per (batch, head, 64-query
// block); nothing is allocated.
tn_status flash64_launch(hipStream_t st, bool f16, int mk, const void* mask, int64_t msb, int64_t msh, int64_t msl,
                         int64_t msk, const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t B, int64_t Hq,
                         int64_t Hkv, int64_t L, int64_t S, float sl2, int causal, uint16_t* out, float* lse) {
    const int64_t nqb = cdiv(L, FA_BQ);
    const int64_t items = B * Hq * nqb;
    if (items > INT32_MAX || B * Hq > INT32_MAX) return fail(TN_EVALUE, "sdpa: shape too large");
    const MaskRef mref{mask, msb, msh, msl, msk};
#define TN_FA64(MK, H)                                                                                           \
    hipLaunchKernelGGL((k_fa64<MK, H>), dim3((unsigned)items), dim3(FA_NT), 0, st, q, k, v, (int)(B * Hq), (int)Hq, \
                       (int)Hkv, (int)L, (int)S, (int)nqb, sl2, causal, out, lse, mref)
    // a mask that varies along the query rows runs on k_flash16 (sdpa.hip):
    // its reads per row do not fit this kernel's 128 registers per wave
    if (mk != 0 && msl != 0) return fail(TN_EINVAL, "flash64: only masks that are the same for every query row");
    if (f16) {
        if (mk == 0) TN_FA64(0, true);
        else if (mk == 1) TN_FA64(1, true);
        else if (mk == 3) TN_FA64(3, true);
        else TN_FA64(2, true);
    } else {
        if (mk == 0) TN_FA64(0, false);
        else if (mk == 1) TN_FA64(1, false);
        else if (mk == 3) TN_FA64(3, false);
        else TN_FA64(2, false);
    }
#undef TN_FA64
    TN_LAUNCHED();
    return TN_OK;
}

}  // namespace tn

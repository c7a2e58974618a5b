// Scaled dot-product attention on gfx950: flash prefill (bf16 and f32) and
// split-KV decode over per-sequence KV caches.
//
// Semantics are the reference's aten._scaled_dot_product_flash_attention_for_cpu
// (torchnative/rust/torch_c/src/aten.rs:10092-10440): softmax(q k^T * scale
// [+ upper-left causal -inf]) v with f32 accumulation, GQA by indexing key/value
// head h / (Hq/Hkv), logsumexp over the masked, scaled scores. The blocked
// online softmax follows the structure of upstream's CPU flash kernel that the
// reference reproduces in flash.rs:587-780 (accumulators rescaled by
// exp(m_old - m_new), P narrowed to the input dtype between the products for
// bf16).
//
// Layout shared by all kernels: scores are computed transposed, S^T = K . Q^T,
// so that in the 16x16 MFMA result layout (lane l holds C[4*(l>>4) + r][l & 15])
// each lane owns one query (column l & 15) and four keys per 16-key tile. Row
// statistics are then in-lane plus two cross-lane steps, and the output is
// accumulated transposed, O^T = V^T . P^T, where the lane's own probabilities
// are directly the B operand and the lane again owns its query's column, so
// the online rescale needs no data movement.
//
// Rescaling is lazy: a row keeps the maximum it last rescaled to until a tile
// raises it by more than 2^8 (in exp2 units), so probabilities stay <= 256 and
// the accumulators are touched only when a wave actually needs it. The result
// is the same softmax; only the common factor differs until the end.
#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <utility>
#include <vector>

#include "tn_common.h"
#include "attn_common.h"
#include "skgeo.h"

namespace tn {
namespace {


// ---------------------------------------------------------------------------
// bf16 prefill on v_mfma_f32_32x32x16_bf16 (the full-rate bf16 MFMA shape).
//
// Workgroup = 2*KG waves over 64 queries of one (batch, head): wave w takes
// query half qw = w & 1 (32 queries) and key group kg = w >> 1. K and V
// stream through a two-stage LDS ring whose stages hold KG*BKW consecutive
// keys; key group kg computes the stage's BKW-key tile kg, so the KG groups
// split the row's keys among themselves and merge through LDS at the end (a
// log2(KG)-round tree). Two waves per SIMD hide each other's MFMA -> softmax
// -> MFMA latency, and a query block's keys are covered KG tiles at a time
// without any traffic outside the CU. Stages are filled with
// buffer_load ... lds: no registers are involved, so the next stage is in
// flight while one is computed, and the stage's position is a scalar buffer
// descriptor, so a stage costs no vector address arithmetic (keys past the
// end read as zero). Rows are stored in 16-byte chunks XOR-swizzled by row so
// that the MFMA operand reads are bank-conflict free. Per tile and wave:
//   S^T = K . Q^T : BKW/32 key halves x D/16 MFMA (A = K rows from LDS, B =
//                   Q^T in registers); lane l owns query l&31, 16 keys per half;
//   P             : exp2(S * scale*log2e - m), narrowed to bf16 (v_cvt_pk_bf16_f32);
//   O^T += V^T P^T: D/32 x BKW/16 MFMA; the V^T operand is read column-wise
//                   from the natural-layout V tile with ds_read_b64_tr_b16.
// K-slot order of a 16-key MFMA step j of key half s: lane half h holds keys
// {32s + 16j + 4h + e, 32s + 16j + 8 + 4h + e : e = 0..3}, which is where the
// 32x32 result layout (lane l holds rows 8(r/4) + 4(l>>5) + r%4) put them.
//
// Long rows are also split across workgroups (the work list, FlashWork,
// balances the items). The splits of a row merge inside this kernel
// (merge_split_rows): each publishes unnormalised (m, l, O) partials with
// device-coherent stores and takes a ticket, and the last one merges them.
// The partials bypass the non-coherent L2, so no device-scope release (which
// writes back the XCD's whole L2) is needed. The softmax runs per 32-key half
// so that one half's products can overlap the other's softmax.
// ---------------------------------------------------------------------------

constexpr int F3_BQ = 64, F3_BK = 64;  // queries per workgroup; key tile of the host-side split unit


// The rows of a split query block, merged inside the prefill kernel. Every
// split item publishes its unnormalised (O, m, l) for the block's rows with
// device-coherent stores (sc1: written through to memory, past this XCD's
// L2), waits until they are acknowledged, and takes a ticket from the block's
// counter. The item that draws the last ticket reads every split's partials
// back with device-coherent loads and merges them in split order -- the same
// arithmetic whichever item finishes last -- then returns the counter to zero
// for the next launch.
// No fence is needed: only the partials cross workgroups, and they never sit
// in a non-coherent cache. The partial stride is nsplit (the launch's
// maximum); rows of the block are contiguous from `row0`.
template <int D, bool F16>
__device__ __attribute__((always_inline)) inline void merge_split_rows(float* part_o, float2* part_ml, uint32_t* tickets, int nsplit,
                                              int split, int ns, int64_t row0, int nrows, int64_t ticket,
                                              bool holder, int r, int hh, const f32x16 (&o)[D / 32], float m,
                                              float l, uint16_t* __restrict__ Og, float* __restrict__ lse,
                                              uint32_t& s_ticket) {
    constexpr uint32_t SC1 = 16;  // cache policy: device scope
    const uint32_t po_bytes = (uint32_t)(nrows * nsplit * D * 4);
    const buf_rsrc ro = make_rsrc(part_o + row0 * nsplit * D, po_bytes);
    const buf_rsrc rm = make_rsrc(part_ml + row0 * nsplit, (uint32_t)(nrows * nsplit * 8));
#if __HIP_DEVICE_COMPILE__
    if (holder) {
        const uint32_t base = (uint32_t)((r * nsplit + split) * D) * 4u;
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
                const u32x4_t v = {__float_as_uint(o[dt][4 * g4]), __float_as_uint(o[dt][4 * g4 + 1]),
                                   __float_as_uint(o[dt][4 * g4 + 2]), __float_as_uint(o[dt][4 * g4 + 3])};
                __builtin_amdgcn_raw_buffer_store_b128(v, ro, base + (uint32_t)(32 * dt + 8 * g4 + 4 * hh) * 4u, 0,
                                                       SC1);
            }
        if (hh == 0) {
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            const u32x2_t v = {__float_as_uint(m), __float_as_uint(l)};
            __builtin_amdgcn_raw_buffer_store_b64(v, rm, (uint32_t)(r * nsplit + split) * 8u, 0, SC1);
        }
    }
#endif
    wait_vmcnt<0>();  // this thread's partials are acknowledged by memory
    __syncthreads();
    if (threadIdx.x == 0) s_ticket = __hip_atomic_fetch_add(tickets + ticket, 1u, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_ticket != (uint32_t)(ns - 1)) return;  // uniform: another split merges the block
#if __HIP_DEVICE_COMPILE__
    // thread -> (row, 4 columns), every split's loads in flight before any is used
    constexpr int TPR = D / 4;
    constexpr int CMAX = 4;
    const int c4 = ((int)threadIdx.x % TPR) * 4;
    for (int rr = (int)threadIdx.x / TPR; rr < nrows; rr += (int)blockDim.x / TPR) {
        typedef float f32x2_t __attribute__((ext_vector_type(2)));
        typedef float f32x4_t __attribute__((ext_vector_type(4)));
        auto ld_ml = [&](int sp) {
            return __builtin_bit_cast(f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
                                                  rm, (uint32_t)(rr * nsplit + sp) * 8u, 0, SC1));
        };
        auto ld_o = [&](int sp) {
            return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                  ro, ((uint32_t)((rr * nsplit + sp) * D + c4)) * 4u, 0, SC1));
        };
        f32x2_t mlv[CMAX];
        f32x4_t pv[CMAX];
#pragma unroll
        for (int sp = 0; sp < CMAX; sp++) {
            mlv[sp] = sp < ns ? ld_ml(sp) : (f32x2_t){-INFINITY, 0.0f};
            pv[sp] = sp < ns ? ld_o(sp) : (f32x4_t){0.f, 0.f, 0.f, 0.f};
        }
        float mm = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < CMAX; sp++) mm = fmaxf(mm, mlv[sp][0]);
        for (int sp = CMAX; sp < ns; sp++) mm = fmaxf(mm, ld_ml(sp)[0]);
        const float mu = (mm == -INFINITY) ? 0.0f : mm;
        float tl = 0.0f, a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        auto add = [&](f32x2_t m_l, f32x4_t v) {
            const float f = exp2f(m_l[0] - mu);
            tl = tl + m_l[1] * f;
            a0 = a0 + v[0] * f;
            a1 = a1 + v[1] * f;
            a2 = a2 + v[2] * f;
            a3 = a3 + v[3] * f;
        };
#pragma unroll
        for (int sp = 0; sp < CMAX; sp++)
            if (sp < ns) add(mlv[sp], pv[sp]);
        for (int sp = CMAX; sp < ns; sp++) add(ld_ml(sp), ld_o(sp));
        const float inv = 1.0f / tl;
        const int64_t row = row0 + rr;
        *reinterpret_cast<uint2*>(Og + row * D + c4) =
            make_uint2(El<F16>::pack_out(a0 * inv, a1 * inv), El<F16>::pack_out(a2 * inv, a3 * inv));
        if (lse && c4 == 0) lse[row] = mm == -INFINITY ? NAN : mu * LN2 + logf(tl);  // a fully masked row is NaN (aten.rs:10392-10420)
    }
#endif
    if (threadIdx.x == 0) __hip_atomic_store(tickets + ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// key groups and keys per wave tile: 32-key wave tiles at both head dims, so
// a ring stage holds 64 keys (16 KB of K and V at D=64, 32 KB at D=128). At
// D=64 this measured 1.5-2% faster on config 2 than 64-key tiles (64 KB of
// ring) and leaves room for more workgroups per CU. One 8-wave workgroup per
// CU measured no faster: its single barrier keeps the two waves of each SIMD
// in the same phase, MFMA against MFMA and softmax against softmax, where
// independent workgroups drift apart and overlap.
template <int D>
struct FlashCfg {
    static constexpr int KG = 2;
    static constexpr int BKW = 32;
};

// A row of n key tiles is cut into row_splits(n, target) items; item s covers
// tiles [s*n/ns, (s+1)*n/ns), so the items differ in size by at most one tile
// and none is empty.
__host__ __device__ inline int row_splits(int n, int target) { return n <= target ? 1 : (n + target - 1) / target; }

// The prefill's work list, passed by value: item classes (query block qt,
// split s) sorted by decreasing size, each class repeated for every (batch,
// head). Workgroup i takes class i / bh, (batch, head) i % bh; consecutive
// workgroups go to the eight XCDs in turn, so every XCD receives the same mix
// of long and short items and the longest start first. ncls = 0: no row is
// split and class c is query block nqb-1-c.
constexpr int FLASH_MAX_CLS = 768;
// A list of at most FLASH_INLINE classes travels inside the kernel arguments,
// so a workgroup's class is one scalar load from the argument segment rather
// than two dependent ones (the table pointer, then the entry).
constexpr int FLASH_INLINE = 128;
struct FlashWork {
    int target;            // tiles per item
    int bh;                // B * Hq
    int ncls;
    const uint32_t* cls;   // device table [ncls] when ncls > FLASH_INLINE: qt | split << 16
    uint32_t inl[FLASH_INLINE];  // the table itself when ncls <= FLASH_INLINE
};

// MASK: 0 none; 1 an f32 additive mask; 2 one in the input format; 3 a bool
// one (MaskRef), added to the scaled scores before the row maximum
// (aten.rs:10383-10389)
template <int D, int MASK = 0, bool F16 = false>
__global__ __launch_bounds__(128 * FlashCfg<D>::KG) void k_flash16(
    const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kg, const uint16_t* __restrict__ Vg, int Hq,
    int Hkv, int L, int S, float sl2, int causal, const FlashWork work, int nsplit, uint16_t* __restrict__ Og,
    float* __restrict__ lse, float* __restrict__ part_o, float2* __restrict__ part_ml, uint32_t* __restrict__ tickets,
    const MaskRef mask) {
    constexpr int KG = FlashCfg<D>::KG;        // key groups
    constexpr int BKW = FlashCfg<D>::BKW;      // keys per wave tile
    constexpr int NH = BKW / 32;               // 32-key halves per wave tile
    constexpr int NW = 2 * KG;                 // waves
    constexpr int NT = 64 * NW;                // threads
    constexpr int ROWS = KG * BKW;             // keys per ring stage
    constexpr int STAGE = ROWS * D;            // elements of one K (or V) stage
    constexpr int CPR = D / 8;                 // 16-byte chunks per row
    constexpr int LPT = ROWS * CPR / NT;       // 16-byte loads per thread per stage, for K and for V each
    static_assert(LPT * NT == ROWS * CPR, "stage must split evenly over the threads");
    // one LDS object per ring stage: with the stage known at compile time the
    // compiler can prove a read of stage s does not alias the loads still
    // landing in the other stage, and inserts no blanket vmcnt(0)
    __shared__ __align__(16) uint16_t sK0[STAGE], sK1[STAGE];
    __shared__ __align__(16) uint16_t sV0[STAGE], sV1[STAGE];
    __shared__ float2 s_ml[KG / 2][2][64];
    __shared__ uint32_t s_ticket;
    auto stK = [&](auto sc) -> uint16_t* {
        if constexpr (decltype(sc)::value == 0) return sK0; else return sK1;
    };
    auto stV = [&](auto sc) -> uint16_t* {
        if constexpr (decltype(sc)::value == 0) return sV0; else return sV1;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, kept in a scalar register
    const int qw = w & 1, kg = w >> 1;                       // query half, key group
    const int lq = lane & 31, hh = lane >> 5;
    const int nqb = (L + F3_BQ - 1) / F3_BQ;
    const int cidx = (int)blockIdx.x / work.bh;
    const int bh = (int)blockIdx.x % work.bh;
    const uint32_t cl = work.ncls == 0              ? (uint32_t)(nqb - 1 - cidx)
                        : work.ncls <= FLASH_INLINE ? work.inl[cidx]
                                                    : work.cls[cidx];
    const int qt = (int)(cl & 0xffffu), split = (int)(cl >> 16);
    const int h = bh % Hq, b = bh / Hq;
    const int kvh = h / (Hq / Hkv);
    const int q0 = qt * F3_BQ;
    const int qw0 = q0 + qw * 32;            // first query of this wave
    const int qi = qw0 + lq;
    const int kend = causal ? min(S, q0 + F3_BQ) : S;
    const int ntiles_row = (kend + F3_BK - 1) / F3_BK;
    const int nsplit_row = row_splits(ntiles_row, work.target);
    const int k_lo = split * ntiles_row / nsplit_row * F3_BK;         // this item's keys: [k_lo, k_hi)
    const int k_hi = min(kend, (split + 1) * ntiles_row / nsplit_row * F3_BK);
    const int nst = (k_hi - k_lo + ROWS - 1) / ROWS;                  // ring stages of this item

    const uint16_t* qp = Qg + ((int64_t)b * Hq + h) * L * D;
    const uint16_t* kp = Kg + ((int64_t)b * Hkv + kvh) * S * D;
    const uint16_t* vp = Vg + ((int64_t)b * Hkv + kvh) * S * D;

    // physical 16-byte chunk of logical chunk c in row r (an involution; it
    // depends on r mod 16 only, so a tile's rows and the stage's rows agree)
    auto swz = [](int r, int c) { return D == 64 ? (c ^ ((r >> 1) & 7)) : (c ^ (r & 15)); };

    using E = El<F16>;
    using V8 = typename E::v8;
    V8 qf[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; c++) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (qi < L) v = *reinterpret_cast<const uint4*>(qp + (int64_t)qi * D + 16 * c + 8 * hh);
        qf[c] = __builtin_bit_cast(V8, v);
    }

    // this lane's byte offset in a stage for its i-th 16-byte load: LDS
    // position p = tid + NT*i (wave w's i-th load covers positions
    // (w + NW*i)*64 .. +63) holds logical chunk swz(row, p % CPR) of row p / CPR
    uint32_t voff[LPT];
#pragma unroll
    for (int i = 0; i < LPT; i++) {
        const int p = tid + NT * i;
        const int row = p / CPR;
        voff[i] = (uint32_t)(row * D + swz(row, p % CPR) * 8) * 2u;
    }
    auto issue = [&](auto sc, int st) {
        const int k0 = k_lo + st * ROWS;
        const uint32_t bytes = (uint32_t)(S - k0) * (uint32_t)(D * 2);  // keys k0 .. S-1
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

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    issue(I0{}, 0);  // nst >= 1: every item has at least one key

    // ring stage sc holds stage st: wait for it, open the other stage (read in
    // the previous step) to the next stage's loads, compute this wave's tile
    auto step = [&](auto sc, int st) {
        wait_vmcnt<0>();  // the only loads in flight are this stage's
        // a bare barrier (no fence: a fence would also wait for the scalar
        // loads); the empty asm statements keep the compiler from moving LDS
        // accesses across it
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (st + 1 < nst) issue(std::integral_constant<int, 1 - decltype(sc)::value>{}, st + 1);

        const int k0 = k_lo + st * ROWS + kg * BKW;
        // past the item's keys, or every query of the wave precedes the tile
        if (k0 >= k_hi || (causal && qw0 + 31 < k0)) return;
        // this wave's tile is rows BKW*kg .. BKW*kg + BKW-1 of the stage; the
        // key group enters through the row index (not the pointer), which
        // keeps the reads attributable to their stage's LDS object, so the
        // compiler does not make them wait for the other stage's loads
        const uint16_t* tK = stK(sc);
        const uint16_t* tV = stV(sc);
        const int kr = BKW * kg;

        float sv[NH][16];
#pragma unroll
        for (int s2 = 0; s2 < NH; s2++) {
            f32x16 acc;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = 0.0f;
            const int row = kr + 32 * s2 + lq;
#pragma unroll
            for (int c = 0; c < D / 16; c++) {
                const V8 ka = *reinterpret_cast<const V8*>(tK + row * D + swz(row, 2 * c + hh) * 8);
                acc = E::mfma(ka, qf[c], acc);
            }
            // The scores are read by VALU next, on interior tiles right after
            // the branch around the edge masking; there the compiler's hazard
            // pass (with MFMA results in VGPRs) emitted no wait states, and
            // the row maximum read a partly accumulated result (wrong, and
            // exp2 overflowed, for large scores). A VALU read of a 16-pass
            // XDL result needs 18 wait states: they are spelled out here,
            // tied to the accumulator so that no read is scheduled above them.
            asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(acc));
#pragma unroll
            for (int r = 0; r < 16; r++) sv[s2][r] = acc[r];
        }
        // Online softmax per 32-key half: the half-1 S products (issued above)
        // run on the matrix core while half 0's softmax runs on the VALU, and
        // half 0's P.V products while half 1's softmax runs.
        const bool edge = k0 + BKW > S || (causal && k0 + BKW - 1 > qw0);
        const float scl = MASK ? 1.0f : sl2;  // scores' factor to log2 units
        // V^T operand rows for this lane's 16-lane group: d = 32dt + 16*((lane>>4)&1) + (lane&15)
        const int gi = lane & 15;
        const int dcol = 16 * ((lane >> 4) & 1) + 4 * (gi & 3);  // source lane's 4 columns
#pragma unroll
        for (int s2 = 0; s2 < NH; s2++) {
            float* v = sv[s2];
            if constexpr (MASK != 0) {
                // scores to log2 units with the mask added: raw*scale*log2e + mask*log2e;
                // from here on the scale is 1
                if (qi < L) {
                    const int64_t mrow = (int64_t)b * mask.sb + (int64_t)h * mask.sh + (int64_t)qi * mask.sl;
#pragma unroll
                    for (int rq = 0; rq < 4; rq++) {
                        const f32x4 mv = mask_quad<MASK, F16>(mask, mrow, k0 + 32 * s2 + 8 * rq + 4 * hh, S);
#pragma unroll
                        for (int e = 0; e < 4; e++) v[4 * rq + e] = v[4 * rq + e] * sl2 + mv[e] * LOG2E;
                    }
                }
            }
            if (edge) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = k0 + 32 * s2 + 8 * (r >> 2) + 4 * hh + (r & 3);
                    if (key >= S || (causal && key > qi)) v[r] = -INFINITY;
                }
            }
            // half maximum: two independent max3 chains over 8 scores each
            float a = max3f(v[0], v[1], v[2]);
            a = max3f(a, v[3], v[4]);
            a = max3f(a, v[5], v[6]);
            float bm = max3f(v[8], v[9], v[10]);
            bm = max3f(bm, v[11], v[12]);
            bm = max3f(bm, v[13], v[14]);
            float mx = max3f(max3f(a, v[7], v[15]), bm, bm);
            mx = xor32_max(mx) * scl;
            const bool need = mx > m + RESCALE_SLACK;
            if (__any(need)) {
                const float mn = need ? mx : m;
                // a row with no key seen yet keeps m = mn = -inf: alpha 1, not 2^NaN
                const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
                l = l * alpha;
#pragma unroll
                for (int i = 0; i < D / 32; i++) o[i] = o[i] * alpha;
                m = mn;
            }
            const float mu = (m == -INFINITY) ? 0.0f : m;
            float p[16];
#pragma unroll
            for (int r = 0; r < 16; r++) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[r], scl, -mu));
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r += 4) ps = ps + ((p[r] + p[r + 1]) + (p[r + 2] + p[r + 3]));
            l = l + ps;
            V8 pf[2];
#pragma unroll
            for (int j = 0; j < 2; j++)
                pf[j] = __builtin_bit_cast(
                    V8, make_uint4(E::pack_p(p[8 * j], p[8 * j + 1]), E::pack_p(p[8 * j + 2], p[8 * j + 3]),
                                   E::pack_p(p[8 * j + 4], p[8 * j + 5]), E::pack_p(p[8 * j + 6], p[8 * j + 7])));
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int r0 = kr + 32 * s2 + 16 * j + 4 * hh + (gi >> 2);
                    const int r1 = r0 + 8;
                    const int col = 32 * dt + dcol;
                    const uint2 lo = lds_read_tr16(tV + r0 * D + swz(r0, col >> 3) * 8 + (col & 7));
                    const uint2 hi = lds_read_tr16(tV + r1 * D + swz(r1, col >> 3) * 8 + (col & 7));
                    const V8 va = __builtin_bit_cast(V8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                    o[dt] = E::mfma(va, pf[j], o[dt]);
                }
            }
        }
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
    // Tree merge of the key groups through LDS: in the round of width `half`,
    // group kg + half hands its (m, l, O) to group kg. Lane l of wave (qw, g)
    // holds the same (query, d) entries for every g. The O buffers of a round
    // take 2*half wave slots of D*128 bytes, laid over the ring arrays (every
    // load has landed and been read once the first barrier has passed).
    constexpr int WSLOT = D / 32 * 16 * 64;        // floats per wave slot
    constexpr int PER_ARR = STAGE / 2 / WSLOT;     // wave slots per ring array
    static_assert(PER_ARR >= 1 && KG <= 4 * PER_ARR, "merge slots must fit in the ring");
#pragma unroll
    for (int half = KG / 2; half >= 1; half /= 2) {
        __syncthreads();
        if (kg >= half && kg < 2 * half) {
            const int x = (kg - half) * 2 + qw;  // wave slot
            float* arr = reinterpret_cast<float*>(x / PER_ARR == 0 ? sK0 : x / PER_ARR == 1 ? sK1
                                                  : x / PER_ARR == 2 ? sV0 : sV1);
            float* xo = arr + (x % PER_ARR) * WSLOT;
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) xo[(dt * 16 + r) * 64 + lane] = o[dt][r];
            s_ml[kg - half][qw][lane] = make_float2(m, l);
        }
        __syncthreads();
        if (kg < half) {
            const int x = kg * 2 + qw;
            const float* arr = reinterpret_cast<const float*>(x / PER_ARR == 0 ? sK0 : x / PER_ARR == 1 ? sK1
                                                              : x / PER_ARR == 2 ? sV0 : sV1);
            const float* xo = arr + (x % PER_ARR) * WSLOT;
            const float2 ml1 = s_ml[kg][qw][lane];
            const float mm = fmaxf(m, ml1.x);
            const float mu = (mm == -INFINITY) ? 0.0f : mm;
            const float a0 = __builtin_amdgcn_exp2f(m - mu);
            const float a1 = __builtin_amdgcn_exp2f(ml1.x - mu);
            l = l * a0 + ml1.y * a1;
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dt][r] = o[dt][r] * a0 + xo[(dt * 16 + r) * 64 + lane] * a1;
            m = mm;
        }
    }
    const int64_t row = ((int64_t)b * Hq + h) * L + qi;
    if (nsplit_row > 1) {
        merge_split_rows<D, F16>(part_o, part_ml, tickets, nsplit, split, nsplit_row, (int64_t)bh * L + q0,
                            min(F3_BQ, L - q0), bh * nqb + qt, kg == 0 && qi < L, qi - q0, hh, o, m, l, Og, lse,
                            s_ticket);
        return;
    }
    if (kg != 0 || qi >= L) return;
    const float inv = 1.0f / l;
    uint16_t* op = Og + row * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++)
            // O^T[d = 32dt + 8g4 + 4hh + e][q = lq]
            *reinterpret_cast<uint2*>(op + 32 * dt + 8 * g4 + 4 * hh) =
                make_uint2(E::pack_out(o[dt][4 * g4] * inv, o[dt][4 * g4 + 1] * inv),
                           E::pack_out(o[dt][4 * g4 + 2] * inv, o[dt][4 * g4 + 3] * inv));
    if (lse && hh == 0) lse[row] = m == -INFINITY ? NAN : m * LN2 + logf(l);
}

// ---------------------------------------------------------------------------
// Any head dimension up to ANY_DMAX other than the MFMA kernels' 64 and 128,
// and a scale of either sign: a plain f32 kernel for every input dtype.
// Workgroup = 256 threads over ANY_BQ = 32 queries of one (batch, head): thread
// (row r = tid / 8, lane t = tid % 8) scores keys t, t + 8, t + 16, t + 24 of
// each 32-key tile with a sequential f32 dot over d, and accumulates output
// columns t, t + 8, ... of its row. K and V tiles are widened to f32 into
// LDS; the row's eight threads share max and sum by shuffles and the row's
// probabilities through LDS. Online softmax in log2 units over the scaled
// scores (so the scale's sign does not matter); probabilities stay f32; the
// output is narrowed RNE to the input dtype.
// ---------------------------------------------------------------------------
constexpr int ANY_DMAX = 256, ANY_BQ = 32;

// element type ET: 0 f32, 1 bf16, 2 f16, 3 f64; arithmetic in f64 for f64
// inputs (the reference computes f64 attention in f64), f32 otherwise
template <int ET>
using AnyT = typename std::conditional<ET == 3, double, float>::type;

template <int ET>
__device__ inline AnyT<ET> any_load(const void* p, int64_t i) {
    if constexpr (ET == 0) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (ET == 1) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else if constexpr (ET == 2) return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else return reinterpret_cast<const double*>(p)[i];
}

template <int ET>
__device__ inline void any_store(void* p, int64_t i, AnyT<ET> v) {
    if constexpr (ET == 0) reinterpret_cast<float*>(p)[i] = v;
    else if constexpr (ET == 1) reinterpret_cast<uint16_t*>(p)[i] = bf16_from_f32(v);
    else if constexpr (ET == 2) reinterpret_cast<uint16_t*>(p)[i] = f16_from_f32(v);
    else reinterpret_cast<double*>(p)[i] = v;
}

// lens (decode): nullable device int32 [B]; sequence b then attends keys
// 0 .. min(lens[b], max_len) - 1 of its S = cap rows. lse is f32, or f64 for
// f64 inputs. Key tiles are 32 keys (16 for f64, which doubles the LDS).
// MASK: 0 none; 1 f32; 2 the query's dtype; 3 bool (MaskRef)
template <int ET, int MASK>
__global__ __launch_bounds__(256) void k_attn_any(const void* __restrict__ Qg, const void* __restrict__ Kg,
                                                  const void* __restrict__ Vg, int Hq, int Hkv, int L, int S, int D,
                                                  double scale, int causal, void* __restrict__ Og,
                                                  void* __restrict__ lse, const MaskRef mask,
                                                  const int32_t* __restrict__ lens, int max_len) {
    using T = AnyT<ET>;
    constexpr int BK = ET == 3 ? 16 : 32;  // keys per tile
    constexpr int KPT = BK / 8;            // keys per thread per tile
    __shared__ T sQ[ANY_BQ * ANY_DMAX];
    __shared__ T sK[BK * (ANY_DMAX + 1)];  // rows padded by one element: the 8 keys a row reads at one d
    __shared__ T sV[BK * ANY_DMAX];        // sit in different banks
    __shared__ T sP[ANY_BQ][BK];
    const T sl2 = (T)scale * (T)1.4426950408889634;  // scores to log2 units
    const T log2e = (T)1.4426950408889634;
    const int tid = threadIdx.x, r = tid >> 3, t = tid & 7;
    const int q0 = blockIdx.x * ANY_BQ, h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (Hq / Hkv);
    const int qi = q0 + r;
    const int64_t bh = (int64_t)b * Hq + h;
    const int64_t qbase = bh * L * D;
    const int64_t kbase = ((int64_t)b * Hkv + kvh) * S * D;
    const int KP = D + 1;
    for (int e = tid; e < ANY_BQ * D; e += 256) {
        const int rr = e / D, d = e - rr * D;
        sQ[rr * D + d] = q0 + rr < L ? any_load<ET>(Qg, qbase + (int64_t)(q0 + rr) * D + d) : (T)0;
    }
    constexpr int NC = ANY_DMAX / 8;  // output columns per thread, at most
    T o[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) o[c] = 0;
    T m = -INFINITY, l = 0;
    // keys this workgroup's rows may see: [0, kvalid)
    const int kvalid = lens ? max(0, min(min(lens[b], max_len), S)) : S;
    const int kend = causal ? min(kvalid, q0 + ANY_BQ) : kvalid;
    for (int k0 = 0; k0 < kend; k0 += BK) {
        __syncthreads();  // the previous tile's reads are done
        for (int e = tid; e < BK * D; e += 256) {
            const int j = e / D, d = e - j * D;
            const bool in = k0 + j < S;
            sK[j * KP + d] = in ? any_load<ET>(Kg, kbase + (int64_t)(k0 + j) * D + d) : (T)0;
            sV[j * D + d] = in ? any_load<ET>(Vg, kbase + (int64_t)(k0 + j) * D + d) : (T)0;
        }
        __syncthreads();
        T sc[KPT];
        T mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            const int j = t + 8 * i, key = k0 + j;
            T acc = 0;
            for (int d = 0; d < D; d++) acc = acc + sQ[r * D + d] * sK[j * KP + d];
            T v = acc * sl2;
            if constexpr (MASK != 0) {
                if (qi < L && key < S) {
                    const int64_t off = (int64_t)b * mask.sb + (int64_t)h * mask.sh + (int64_t)qi * mask.sl +
                                        (int64_t)key * mask.sk;
                    T mv;
                    if constexpr (MASK == 1) mv = (T)reinterpret_cast<const float*>(mask.p)[off];
                    else if constexpr (MASK == 3) mv = reinterpret_cast<const uint8_t*>(mask.p)[off] ? (T)0 : (T)-INFINITY;
                    else mv = any_load<ET>(mask.p, off);
                    v = v + mv * log2e;
                }
            }
            if (key >= kvalid || (causal && key > qi)) v = -INFINITY;
            sc[i] = v;
            mx = fmax(mx, v);
        }
        mx = fmax(mx, __shfl_xor(mx, 1));
        mx = fmax(mx, __shfl_xor(mx, 2));
        mx = fmax(mx, __shfl_xor(mx, 4));
        const T mn = fmax(m, mx);
        const T alpha = mn == -INFINITY ? (T)1 : exp2(m - mn);
        const T mu = mn == -INFINITY ? (T)0 : mn;
        T ps = 0;
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            const T p = exp2(sc[i] - mu);
            sP[r][t + 8 * i] = p;
            ps = ps + p;
        }
        ps = ps + __shfl_xor(ps, 1);
        ps = ps + __shfl_xor(ps, 2);
        ps = ps + __shfl_xor(ps, 4);
        l = l * alpha + ps;
        m = mn;
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int d = t + 8 * c;
            if (d < D) {
                T acc = o[c] * alpha;
                for (int j = 0; j < BK; j++) acc = acc + sP[r][j] * sV[j * D + d];
                o[c] = acc;
            }
        }
    }
    if (qi >= L) return;
    const T inv = (T)1 / l;  // a row with no key: 0 * inf = NaN, as the reference's (aten.rs:10392-10420)
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int d = t + 8 * c;
        if (d < D) any_store<ET>(Og, qbase + (int64_t)qi * D + d, o[c] * inv);
    }
    // a row with no key: NaN, as the reference's (aten.rs:10392-10420); a decode
    // sequence of length 0: -inf, as the split decode kernels give
    if (lse && t == 0) {
        const T lv = m == -INFINITY ? (lens ? (T)-INFINITY : (T)NAN) : m * (T)0.69314718055994531 + log(l);
        if constexpr (ET == 3) reinterpret_cast<double*>(lse)[bh * L + qi] = lv;
        else reinterpret_cast<float*>(lse)[bh * L + qi] = lv;
    }
}

// Eight waves per workgroup: each K/V tile staged in LDS serves 128 queries
// (half the staging per product of a four-wave workgroup). At 121-149 VGPRs
// two such workgroups share a CU.
constexpr int PF_WAVES = 8, PF_THREADS = 64 * PF_WAVES;
constexpr int PF_BQ = 16 * PF_WAVES, PF_BK = 64;


// ---------------------------------------------------------------------------
// f32 prefill: the same decomposition on v_mfma_f32_16x16x4_f32 (K = 4 per op).
// The head dim is permuted inside each product so that every operand a lane
// needs is contiguous in LDS and comes in 16-byte reads:
//   S^T : product c sums d = 16g + c over lane groups g (g = lane >> 4), so
//         lane (key lq, g) feeds K[key][16g + c] for c = 0..15: its 16 K
//         operands of a 16-key slice are four ds_read_b128; Q^T likewise from
//         registers (q[16g + c]).
//   O^T : output tile dt holds d = 4i + dt in its row i, so for key slot r of
//         slice kt lane (lq, g) feeds V[16kt + 4g + r][4lq + dt], dt = 0..3:
//         one ds_read_b128 serves all four tiles; lane (q, g) ends up holding
//         d = 16g .. 16g + 15 of query q.
// The next slice's K operands are read while the current slice's products
// run. Row strides are padded to 4 mod 32 dwords, so each 8-lane phase of a
// 16-byte read covers all 32 banks.
// ---------------------------------------------------------------------------

// MASK: 1 adds an f32 mask, 3 a bool one (MaskRef), to the scaled scores
// (aten.rs:10383-10389)
template <int D, int BK, int MASK = 0>
__global__ __launch_bounds__(PF_THREADS) void k_fa_f32(const float* __restrict__ Qg, const float* __restrict__ Kg,
                                              const float* __restrict__ Vg, int Hq, int Hkv, int L, int S,
                                              float sl2, int causal, const SkGeo geo,
                                              float* __restrict__ Og, float* __restrict__ lse,
                                              float* __restrict__ part_o, float2* __restrict__ part_ml,
                                              uint32_t* __restrict__ tickets, const MaskRef mask) {
    constexpr int BQ = PF_BQ;
    constexpr int RS = D + 4;
    constexpr int CH = (BK * D / 4) / PF_THREADS;  // float4 chunks of K (and of V) per thread
    static_assert(CH * PF_THREADS == BK * D / 4, "tile staging");
    __shared__ __align__(16) float sK[2][BK * RS];
    __shared__ __align__(16) float sV[2][BK * RS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    // consecutive ranges on one XCD: a head's K and V fetched into one or two L2s
    const int64_t gw = geo.xcd_order(blockIdx.x);
    const int64_t u_hi = geo.lo(gw + 1);

    // query block qt of (batch, head) bh, key tiles t_begin .. t_end-1;
    // slot < 0: the whole block, written to the output
    __shared__ uint32_t s_ticket;
    auto block = [&](int64_t bh, int qt, int t_begin, int t_end, int slot, int64_t u0) __attribute__((always_inline)) {
        const int h = (int)(bh % Hq), b = (int)(bh / Hq);
        const int kvh = h / (Hq / Hkv);
        const int q0 = qt * BQ;
        const int qi = q0 + w * 16 + lq;
        const float* qp = Qg + ((int64_t)b * Hq + h) * L * D;
        const float* kp = Kg + ((int64_t)b * Hkv + kvh) * S * D;
        const float* vp = Vg + ((int64_t)b * Hkv + kvh) * S * D;

            // q[16g + c] for the D/16 row slices of 16: slice e holds d = 64e + 16g + c
            constexpr int DS = D / 64;  // 64-wide slices of the head dim
            static_assert(D % 64 == 0, "head dim");
            float qf[DS][16];
        #pragma unroll
            for (int e = 0; e < DS; e++)
        #pragma unroll
                for (int c4 = 0; c4 < 4; c4++) {
                    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (qi < L) v = *reinterpret_cast<const float4*>(qp + (int64_t)qi * D + 64 * e + 16 * g + 4 * c4);
                    qf[e][4 * c4] = v.x;
                    qf[e][4 * c4 + 1] = v.y;
                    qf[e][4 * c4 + 2] = v.z;
                    qf[e][4 * c4 + 3] = v.w;
                }
            // o[e][dt] row i holds d = 64e + 4i + dt
            f32x4 o[DS][4];
        #pragma unroll
            for (int e = 0; e < DS; e++)
        #pragma unroll
                for (int i = 0; i < 4; i++) o[e][i] = (f32x4){0.f, 0.f, 0.f, 0.f};
            float m = -INFINITY, l = 0.0f;

            float4 kr[CH], vr[CH];
            auto gload = [&](int k0) {
        #pragma unroll
                for (int it = 0; it < CH; it++) {
                    const int c = tid + it * PF_THREADS;
                    const int r = c / (D / 4), part = c % (D / 4);
                    kr[it] = vr[it] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (k0 + r < S) {
                        kr[it] = *reinterpret_cast<const float4*>(kp + (int64_t)(k0 + r) * D + part * 4);
                        vr[it] = *reinterpret_cast<const float4*>(vp + (int64_t)(k0 + r) * D + part * 4);
                    }
                }
            };
            auto lstore = [&](int buf) {
        #pragma unroll
                for (int it = 0; it < CH; it++) {
                    const int c = tid + it * PF_THREADS;
                    const int r = c / (D / 4), part = c % (D / 4);
                    *reinterpret_cast<float4*>(&sK[buf][r * RS + part * 4]) = kr[it];
                    *reinterpret_cast<float4*>(&sV[buf][r * RS + part * 4]) = vr[it];
                }
            };
            // lane (lq, g)'s K operands of slice kt, head-dim slice e: K[16kt + lq][64e + 16g .. +15]
            auto kread = [&](int buf, int kt, int e, float4* kf) __attribute__((always_inline)) {
                const float* kp4 = &sK[buf][(16 * kt + lq) * RS + 64 * e + 16 * g];
        #pragma unroll
                for (int j = 0; j < 4; j++) kf[j] = *reinterpret_cast<const float4*>(kp4 + 4 * j);
            };

            gload(t_begin * BK);
            lstore(0);
            __syncthreads();
            for (int t = t_begin; t < t_end; t++) {
                const int buf = (t - t_begin) & 1;
                const int k0 = t * BK;
                if (t + 1 < t_end) gload(k0 + BK);

                f32x4 s[BK / 16];
                float4 kf[2][4];
                kread(buf, 0, 0, kf[0]);
        #pragma unroll
                for (int kt = 0; kt < BK / 16; kt++) {
                    s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        #pragma unroll
                    for (int e = 0; e < DS; e++) {
                        const int cur = (kt * DS + e) & 1;
                        // the next slice's operands while these products run
                        if (e + 1 < DS) kread(buf, kt, e + 1, kf[cur ^ 1]);
                        else if (kt + 1 < BK / 16) kread(buf, kt + 1, 0, kf[cur ^ 1]);
        #pragma unroll
                        for (int j = 0; j < 4; j++) {
                            s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[cur][j].x, qf[e][4 * j], s[kt], 0, 0, 0);
                            s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[cur][j].y, qf[e][4 * j + 1], s[kt], 0, 0, 0);
                            s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[cur][j].z, qf[e][4 * j + 2], s[kt], 0, 0, 0);
                            s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[cur][j].w, qf[e][4 * j + 3], s[kt], 0, 0, 0);
                        }
                    }
                }
                if constexpr (MASK != 0) {
                    // scores to log2 units with the mask added; from here on the scale is 1
                    if (qi < L) {
                        const int64_t mrow = (int64_t)b * mask.sb + (int64_t)h * mask.sh + (int64_t)qi * mask.sl;
        #pragma unroll
                        for (int kt = 0; kt < BK / 16; kt++) {
                            const f32x4 mv = mask_quad<MASK, false>(mask, mrow, k0 + 16 * kt + 4 * g, S);
        #pragma unroll
                            for (int r = 0; r < 4; r++) s[kt][r] = s[kt][r] * sl2 + mv[r] * LOG2E;
                        }
                    }
                }
                const float scl = MASK ? 1.0f : sl2;  // scores' factor to log2 units
                if (k0 + BK > S || (causal && k0 + BK - 1 > q0 + w * 16)) {
        #pragma unroll
                    for (int kt = 0; kt < BK / 16; kt++)
        #pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int key = k0 + 16 * kt + 4 * g + r;
                            if (key >= S || (causal && key > qi)) s[kt][r] = -INFINITY;
                        }
                }
                float mx = -INFINITY;
        #pragma unroll
                for (int kt = 0; kt < BK / 16; kt++)
                    mx = fmaxf(mx, fmaxf(fmaxf(s[kt][0], s[kt][1]), fmaxf(s[kt][2], s[kt][3])));
                mx = wave_xor_max(mx) * scl;
                const bool need = mx > m + RESCALE_SLACK;
                if (__any(need)) {
                    const float mn = need ? mx : m;
                    const float alpha = mn == -INFINITY ? 1.0f : exp2f(m - mn);  // no key seen yet: 1, not 2^NaN
                    l = l * alpha;
        #pragma unroll
                    for (int e = 0; e < DS; e++)
        #pragma unroll
                        for (int i = 0; i < 4; i++) o[e][i] = o[e][i] * alpha;
                    m = mn;
                }
                const float mu = (m == -INFINITY) ? 0.0f : m;
                // lane (lq, g)'s V operands of key slot (kt, r): V[16kt + 4g + r][64e + 4lq .. +3]
                auto vread = [&](int kt, int r, float4* vv) __attribute__((always_inline)) {
                    const float* vrow = &sV[buf][(16 * kt + 4 * g + r) * RS + 4 * lq];
        #pragma unroll
                    for (int e = 0; e < DS; e++) vv[e] = *reinterpret_cast<const float4*>(vrow + 64 * e);
                };
                float4 vv[2][DS];
                vread(0, 0, vv[0]);
        #pragma unroll
                for (int kt = 0; kt < BK / 16; kt++) {
        #pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int cur = (4 * kt + r) & 1;
                        // the next key slot's operands while these products run
                        if (4 * kt + r + 1 < BK / 4) vread((4 * kt + r + 1) >> 2, (r + 1) & 3, vv[cur ^ 1]);
                        // exp2 of a value <= RESCALE_SLACK; v_exp_f32 flushes results
                        // below 2^-126 to zero, a change far below the f32 tolerance
                        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][r], scl, -mu));
                        l = l + p;
        #pragma unroll
                        for (int e = 0; e < DS; e++) {
                            o[e][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[cur][e].x, p, o[e][0], 0, 0, 0);
                            o[e][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[cur][e].y, p, o[e][1], 0, 0, 0);
                            o[e][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[cur][e].z, p, o[e][2], 0, 0, 0);
                            o[e][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[cur][e].w, p, o[e][3], 0, 0, 0);
                        }
                    }
                }
                if (t + 1 < t_end) lstore(buf ^ 1);
                __syncthreads();
            }


        l = wave_xor_sum(l);
        // lane (q, g) holds d = 64e + 16g + 4r + dt in o[e][dt][r]
        if (slot < 0) {
            if (qi >= L) return;
            const int64_t row = bh * L + qi;
            const float inv = 1.0f / l;
            float* op = Og + row * D;
#pragma unroll
            for (int e = 0; e < DS; e++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    *reinterpret_cast<float4*>(op + 64 * e + 16 * g + 4 * r) =
                        make_float4(o[e][0][r] * inv, o[e][1][r] * inv, o[e][2][r] * inv, o[e][3][r] * inv);
            if (lse && g == 0) lse[row] = m == -INFINITY ? NAN : m * LN2 + logf(l);
            return;
        }
        // A cut block: publish this workgroup's (O, m, l) with device-coherent
        // stores (sc1: written through to memory, past this XCD's L2), wait
        // until they are acknowledged, and take a ticket from the block's
        // counter. The workgroup that draws the last ticket reads every
        // partial back with device-coherent loads, merges them in workgroup
        // order and returns the counter to zero for the next launch. No
        // fence is needed: only the partials cross workgroups, and they never
        // sit in a non-coherent cache.
        // A slot's O is kept in register order: store k = 4e + r of wave w is
        // 1 KB at float (w * 4 DS + k) * 256, lane by lane, so every write-
        // through store covers whole lines (row-major rows took 16-byte
        // pieces at a 64-byte stride, which memory saw as partial writes).
        constexpr uint32_t SC1 = 16;  // cache policy: device scope
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const buf_rsrc ro = make_rsrc(part_o, (uint32_t)(2 * geo.G * BQ * D * 4));
        const buf_rsrc rm = make_rsrc(part_ml, (uint32_t)(2 * geo.G * BQ * 8));
#if __HIP_DEVICE_COMPILE__
        {
            const uint32_t prow = (uint32_t)(slot * BQ + w * 16 + lq);
            const uint32_t wbase = (uint32_t)slot * (uint32_t)(BQ * D) + (uint32_t)(w * 4 * DS) * 256u + 4u * lane;
#pragma unroll
            for (int e = 0; e < DS; e++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const u32x4_t v = {__float_as_uint(o[e][0][r]), __float_as_uint(o[e][1][r]),
                                       __float_as_uint(o[e][2][r]), __float_as_uint(o[e][3][r])};
                    __builtin_amdgcn_raw_buffer_store_b128(v, ro, (wbase + (uint32_t)(4 * e + r) * 256u) * 4u, 0, SC1);
                }
            if (g == 0) {
                const u32x2_t v = {__float_as_uint(m), __float_as_uint(l)};
                __builtin_amdgcn_raw_buffer_store_b64(v, rm, prow * 8u, 0, SC1);
            }
        }
#endif
        wait_vmcnt<0>();  // this thread's partials are acknowledged by memory
        const int n = geo.nt(qt);
        const int64_t g_lo = geo.wg_of(u0), g_hi = geo.wg_of(u0 + n - 1);
        const int64_t tk = bh * geo.nqb + qt;
        __syncthreads();
        if (threadIdx.x == 0)
            s_ticket = __hip_atomic_fetch_add(tickets + tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s_ticket != (uint32_t)(g_hi - g_lo)) return;  // uniform: another workgroup merges the block
        // g_lo holds the block in slot 2 g_lo + 1 unless the block is where it
        // started; every later workgroup starts inside the block: slot 2g
        const int64_t s_lo = 2 * g_lo + (geo.lo(g_lo) < u0 ? 1 : 0);
        const int np = (int)(g_hi - g_lo + 1);
#if __HIP_DEVICE_COMPILE__
        constexpr int CMAX = 8;  // partials whose loads are in flight together
        // item it is float 4 it of a slot in register order: four columns of
        // one row, consecutive threads reading consecutive 16 bytes
        for (int it = tid; it < BQ * D / 4; it += PF_THREADS) {
            const int ln = it & 63, k = (it >> 6) % (4 * DS), wv = (it >> 6) / (4 * DS);
            const int rr = 16 * wv + (ln & 15);
            const int c4 = 64 * (k >> 2) + 16 * (ln >> 4) + 4 * (k & 3);
            const int qrow = qt * BQ + rr;
            if (qrow >= L) continue;
            auto prow_of = [&](int i) { return (uint32_t)((i == 0 ? s_lo : 2 * (g_lo + i)) * BQ + rr); };
            auto slot_of = [&](int i) { return (uint32_t)(i == 0 ? s_lo : 2 * (g_lo + i)); };
            typedef float f32x2_t __attribute__((ext_vector_type(2)));
            typedef float f32x4_t __attribute__((ext_vector_type(4)));
            auto ld_ml = [&](int i) {
                return __builtin_bit_cast(f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rm, prow_of(i) * 8u, 0, SC1));
            };
            auto ld_o = [&](int i) {
                return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                       ro, (slot_of(i) * (uint32_t)(BQ * D) + 4u * it) * 4u, 0, SC1));
            };
            f32x2_t mlv[CMAX];
            f32x4_t pv[CMAX];
#pragma unroll
            for (int i = 0; i < CMAX; i++) {
                mlv[i] = i < np ? ld_ml(i) : (f32x2_t){-INFINITY, 0.0f};
                pv[i] = i < np ? ld_o(i) : (f32x4_t){0.f, 0.f, 0.f, 0.f};
            }
            float mm = -INFINITY;
#pragma unroll
            for (int i = 0; i < CMAX; i++) mm = fmaxf(mm, mlv[i][0]);  // absent partials hold -inf
            for (int i = CMAX; i < np; i++) mm = fmaxf(mm, ld_ml(i)[0]);
            const float mu = (mm == -INFINITY) ? 0.0f : mm;
            float tl = 0.0f, a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            auto add = [&](f32x2_t m_l, f32x4_t v) {
                const float f = exp2f(m_l[0] - mu);
                tl = tl + m_l[1] * f;
                a0 = a0 + v[0] * f;
                a1 = a1 + v[1] * f;
                a2 = a2 + v[2] * f;
                a3 = a3 + v[3] * f;
            };
#pragma unroll
            for (int i = 0; i < CMAX; i++)
                if (i < np) add(mlv[i], pv[i]);
            for (int i = CMAX; i < np; i++) add(ld_ml(i), ld_o(i));
            const float inv = 1.0f / tl;
            const int64_t row = bh * L + qrow;
            *reinterpret_cast<float4*>(Og + row * D + c4) = make_float4(a0 * inv, a1 * inv, a2 * inv, a3 * inv);
            if (lse && c4 == 0) lse[row] = mm == -INFINITY ? NAN : mu * LN2 + logf(tl);
        }
#endif
        if (tid == 0) __hip_atomic_store(tickets + tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    int64_t u = geo.lo(gw);
    bool first = true;
    while (u < u_hi) {  // uniform over the workgroup
        int64_t bh;
        int qt, t0;
        geo.locate(u, bh, qt, t0);
        const int n = geo.nt(qt);
        const int t1 = (int)(t0 + (u_hi - u) < n ? t0 + (u_hi - u) : n);
        block(bh, qt, t0, t1, (t0 == 0 && t1 == n) ? -1 : (int)(2 * gw + (first ? 0 : 1)), u - t0);
        u += t1 - t0;
        first = false;
    }
}

// ---------------------------------------------------------------------------
// Decode (one query token per sequence), bf16, split-KV.
// Grid (splits of 256 keys, Hkv * groups, B); a workgroup of 4 waves covers
// one split of one sequence for NR query heads that share a key/value head;
// each wave takes 64 keys and issues all of its K and V loads at once (32 KB
// per wave at D=128), so the HBM stream is limited by occupancy, not by
// round trips. Per wave:
//   S^T  : MFMA 16x16x32 with K rows straight from HBM (16 B per lane),
//          query columns 0..NR-1 real, the rest zero;
//   P.V  : VALU, lane (key group g = lane>>4, d slice DL*(lane&15)) over its
//          16 V chunks, probabilities broadcast from LDS.
// The four waves merge in LDS and write one (m, l, O) partial per split;
// k_decode_combine merges the splits.
// ---------------------------------------------------------------------------

constexpr int DEC_WAVE_KEYS = 64;
constexpr int DEC_SPLIT = 4 * DEC_WAVE_KEYS;  // keys per workgroup
static_assert(DEC_SPLIT == DECODE_SPLIT_KEYS, "the decode step sizes its partials with this");

template <int D, int NR, bool F16 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_decode_bf16(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
                   int Hq, int Hkv, int nrep, int cap, const int32_t* __restrict__ lens, int nsplit, float sl2,
                   float* __restrict__ part_o, float2* __restrict__ part_ml) {
    static_assert(D == 128 || D == 64, "head dim");
    constexpr int DL = D / 16;  // d values per lane in P.V
    __shared__ float sP[4][NR][DEC_WAVE_KEYS];
    __shared__ float sO[4][NR][D];
    __shared__ float2 sML[4][NR];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    const int groups = nrep / NR;
    const int kvh = blockIdx.y / groups, grp = blockIdx.y % groups;
    const int b = blockIdx.z, split = blockIdx.x;
    int len = lens[b];
    len = len < 0 ? 0 : (len > cap ? cap : len);
    if (split * DEC_SPLIT >= len) return;  // uniform over the workgroup
    const int k0 = split * DEC_SPLIT + w * DEC_WAVE_KEYS;
    const int nk = min(max(len - k0, 0), DEC_WAVE_KEYS);
    const int hq0 = kvh * nrep + grp * NR;
    const uint16_t* kp = Kc + ((int64_t)b * Hkv + kvh) * cap * D;
    const uint16_t* vp = Vc + ((int64_t)b * Hkv + kvh) * cap * D;

    // all loads of this wave up front
    uint4 kf[4][D / 32];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        const int key = 16 * kt + lq;
#pragma unroll
        for (int c = 0; c < D / 32; c++) {
            kf[kt][c] = make_uint4(0, 0, 0, 0);
            if (key < nk) kf[kt][c] = *reinterpret_cast<const uint4*>(kp + (int64_t)(k0 + key) * D + 32 * c + 8 * g);
        }
    }
    typedef typename std::conditional<DL == 8, uint4, uint2>::type vchunk;
    vchunk vv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int kk = 4 * i + g;
        vv[i] = vchunk{};
        if (kk < nk) vv[i] = *reinterpret_cast<const vchunk*>(vp + (int64_t)(k0 + kk) * D + DL * lq);
    }
    typename El<F16>::v8 qf[D / 32];
#pragma unroll
    for (int c = 0; c < D / 32; c++) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (lq < NR) v = *reinterpret_cast<const uint4*>(Qg + ((int64_t)b * Hq + hq0 + lq) * D + 32 * c + 8 * g);
        qf[c] = __builtin_bit_cast(typename El<F16>::v8, v);
    }

    f32x4 s[4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < D / 32; c++)
            s[kt] = El<F16>::mfma16(__builtin_bit_cast(typename El<F16>::v8, kf[kt][c]), qf[c], s[kt]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (16 * kt + 4 * g + r >= nk) s[kt][r] = -INFINITY;
            mx = fmaxf(mx, s[kt][r]);
        }
    const float m = wave_xor_max(mx) * sl2;
    const float mu = (m == -INFINITY) ? 0.0f : m;
    float l = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = exp2f(__builtin_fmaf(s[kt][r], sl2, -mu));
            l = l + p;
            if (lq < NR) sP[w][lq][16 * kt + 4 * g + r] = p;
        }
    l = wave_xor_sum(l);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float o[NR][DL];
#pragma unroll
    for (int hh = 0; hh < NR; hh++)
#pragma unroll
        for (int e = 0; e < DL; e++) o[hh][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int kk = 4 * i + g;
        float vf[DL];
        uint32_t ws[DL / 2];
        __builtin_memcpy(ws, &vv[i], sizeof(ws));
#pragma unroll
        for (int e = 0; e < DL / 2; e++) {
            vf[2 * e] = El<F16>::lo(ws[e]);
            vf[2 * e + 1] = El<F16>::hi(ws[e]);
        }
#pragma unroll
        for (int hh = 0; hh < NR; hh++) {
            const float p = sP[w][hh][kk];  // 0 for keys past the end
#pragma unroll
            for (int e = 0; e < DL; e++) o[hh][e] = __builtin_fmaf(p, vf[e], o[hh][e]);
        }
    }
#pragma unroll
    for (int hh = 0; hh < NR; hh++)
#pragma unroll
        for (int e = 0; e < DL; e++) o[hh][e] = wave_xor_sum(o[hh][e]);
    if (g == 0) {
#pragma unroll
        for (int hh = 0; hh < NR; hh++)
#pragma unroll
            for (int e = 0; e < DL; e += 4)
                *reinterpret_cast<float4*>(&sO[w][hh][DL * lq + e]) =
                    make_float4(o[hh][e], o[hh][e + 1], o[hh][e + 2], o[hh][e + 3]);
        if (lq < NR) sML[w][lq] = make_float2(m, l);
    }
    __syncthreads();
    // merge the four waves: thread -> (head, d)
    for (int idx = tid; idx < NR * D; idx += 256) {
        const int hh = idx / D, d = idx % D;
        float mm = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) mm = fmaxf(mm, sML[ww][hh].x);
        const float mm_u = (mm == -INFINITY) ? 0.0f : mm;
        float tl = 0.0f, acc = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float f = exp2f(sML[ww][hh].x - mm_u);
            tl = tl + sML[ww][hh].y * f;
            acc = acc + sO[ww][hh][d] * f;
        }
        const int64_t prow = ((int64_t)b * Hq + hq0 + hh) * nsplit + split;
        part_o[prow * D + d] = acc;
        if (d == 0) part_ml[prow] = make_float2(mm, tl);
    }
}

// ---------------------------------------------------------------------------
// Decode, bf16, stream-K over the cached keys of every sequence.
// A segment is one (sequence b, kv head, group of NR query heads): its keys
// are ceil(len_b / 16) units of 16. Laid end to end, the segments are cut
// into W equal unit ranges, one per wave of a persistent grid, so every wave
// streams the same number of bytes whatever the length mix. A wave walks its
// range in chunks of up to 32 keys with the next chunk's K, V and q loads in
// flight while it computes the current one (raw buffer loads whose range ends
// at the segment's last key, so keys past it read as zero without a branch),
// keeps an online softmax per query head, and writes one unnormalised
// (O, m, l) partial each time its range leaves a segment. The partial of
// (segment s, wave w) goes to slot s + w: walking the keys in order, neither
// s nor w decreases and one of them grows, so the slots are distinct and fewer
// than #segments + W. k_decode_sk_combine merges a segment's partials in wave
// order. No barrier: every wave works alone.
//   S^T : MFMA 16x16x32, A = K rows (lane: key lq, d 32c + 8g .. +7), B = q^T;
//         lane l holds the scores of keys 16kt + 4g + r for head lq.
//   P.V : VALU, lane (g, d slice DL*lq) over the same keys 16kt + 4g + r, whose
//         probabilities for head h sit in lane 16g + h of the lane's own
//         16-lane row: a DPP row_newbcast broadcasts them.
// Scores are scaled before the row maximum, so any sign of scale is right.
// ---------------------------------------------------------------------------
constexpr int SK_UNIT = 16;    // keys per unit of the partition
constexpr int SK_MAXB = 1024;  // sequences whose prefix sums a workgroup keeps in LDS
// units per chunk and chunks in the register ring, by head dim: a ring slot
// holds the chunk's K, V and q (48 VGPRs at D=128 with one unit, 40 at D=64
// with two), and NB - 1 slots are in flight while one is computed
template <int D, int NR>
struct SkCfg {
    static constexpr int CH = D == 128 ? 1 : 2;
    static constexpr int NB = (D == 128 && NR > 4) ? 3 : 4;  // 8 heads' accumulators take a slot's registers
};

template <int D, int NR, bool F16 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_decode_sk_bf16(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kc,
                      const uint16_t* __restrict__ Vc, int B, int Hq, int Hkv, int nrep, int cap,
                      const int32_t* __restrict__ lens, int max_len, float sl2, float* __restrict__ part_o,
                      float2* __restrict__ part_ml, int* __restrict__ pref_out) {
    static_assert(D == 128 || D == 64, "head dim");
    constexpr int DL = D / 16;  // d values per lane in P.V
    constexpr int CH = SkCfg<D, NR>::CH, NB = SkCfg<D, NR>::NB;
    typedef typename std::conditional<DL == 8, uint4, uint2>::type vchunk;
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    __shared__ int s_len[SK_MAXB];
    __shared__ int s_pre[SK_MAXB + 1];  // G * (units of sequences 0 .. b-1); the host checks it fits
    // K of each ring slot, per wave: the chunk's CH * 16 rows, brought in by
    // LDS DMA 1 KB (whole rows) per instruction and read back in the MFMA's
    // layout. Row r's 16-byte chunk c sits at physical chunk c ^ (r % CPR), so
    // the sixteen rows one read instruction touches hit distinct banks. One
    // LDS object per slot lets the compiler tell a read of one slot from the
    // DMA landing in another.
    constexpr int KT_ELEMS = CH * 16 * D;  // 4 KB of K per chunk
    constexpr int CPR = D / 8;             // 16-byte chunks per K row
    __shared__ __align__(16) uint16_t sK0[4][KT_ELEMS], sK1[4][KT_ELEMS], sK2[4][KT_ELEMS], sK3[4][KT_ELEMS];
    static_assert(NB <= 4 && KT_ELEMS * 2 == 4096, "K ring slots");

    const int groups = nrep / NR;
    const int G = Hkv * groups;  // segments per sequence
    // lengths clamped to [0, max_len] (a longer one is truncated) and their
    // prefix sums in units, scaled by the segments per sequence
    for (int i = threadIdx.x; i < B; i += blockDim.x) {
        int len = lens[i];
        s_len[i] = len < 0 ? 0 : (len > max_len ? max_len : len);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        // one wave scans: 64 lanes take consecutive stripes of the sequences
        const int per = (B + 63) / 64;
        const int lo = min(B, (int)threadIdx.x * per), hi = min(B, lo + per);
        int run = 0;
        for (int i = lo; i < hi; i++) run += (s_len[i] + SK_UNIT - 1) / SK_UNIT;
        int inc = run;  // inclusive scan over the lanes
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(inc, off, 64);
            if ((int)threadIdx.x >= off) inc += t;
        }
        int acc = inc - run;
        for (int i = lo; i < hi; i++) {
            s_pre[i] = acc * G;
            acc += (s_len[i] + SK_UNIT - 1) / SK_UNIT;
        }
        if (threadIdx.x == 63) s_pre[B] = inc * G;
    }
    __syncthreads();
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i <= B; i += blockDim.x) pref_out[i] = s_pre[i];

    // values every lane of a wave agrees on, moved to scalar registers so that
    // the buffer descriptors built from them stay scalar
    auto rfl = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    const int lane = threadIdx.x & 63, lq = lane & 15, g = lane >> 4;
    // W = min(waves of the grid, units): every working wave gets at least one
    // unit, so the waves meeting a segment are consecutive
    const int T = rfl(s_pre[B]);
    const int64_t W = min((int64_t)gridDim.x * (blockDim.x >> 6), (int64_t)T);
    const int wv = (int)blockIdx.x * (int)(blockDim.x >> 6) + rfl((int)threadIdx.x >> 6);
    if (wv >= W) return;  // uniform over the wave
    const int u_lo = rfl((int)floordiv_nn((int64_t)wv * T, W)), u_hi = rfl((int)floordiv_nn((int64_t)(wv + 1) * T, W));

    // walking state, uniform over the wave: the segment (b, sg) holding unit u
    int b, sg, n, len, seg0;
    {
        int lo = 0, hi = B;  // largest b with s_pre[b] <= u_lo (s_pre[B] = T > u_lo)
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (rfl(s_pre[mid]) <= u_lo) lo = mid; else hi = mid;
        }
        b = lo;
        len = rfl(s_len[b]);
        n = (len + SK_UNIT - 1) / SK_UNIT;  // > 0: u_lo lies in b's units
        const int pb = rfl(s_pre[b]);
        sg = (u_lo - pb) / n;
        seg0 = pb + sg * n;
    }
    int u = u_lo;

    struct Chunk {
        int b, sg, key0, nk;
        bool last;
    };
    // the next chunk of the range; past its end, an empty chunk (nk = 0) whose
    // loads have a zero-byte range: they read zeros and touch no memory, so
    // every ring step issues the same loads
    auto make = [&]() {
        Chunk c;
        if (u >= u_hi) {
            c.b = 0;
            c.sg = 0;
            c.key0 = 0;
            c.nk = 0;
            c.last = false;
            return c;
        }
        const int seg_end = seg0 + n;
        const int cu = min(CH, min(u_hi - u, seg_end - u));
        c.b = b;
        c.sg = sg;
        c.key0 = (u - seg0) * SK_UNIT;
        c.nk = min(cu * SK_UNIT, len - c.key0);
        c.last = (u + cu == seg_end) || (u + cu == u_hi);
        u += cu;
        if (u == seg_end && u < u_hi) {  // on to the next segment that has keys
            if (++sg == G) {
                sg = 0;
                do {
                    ++b;
                    len = rfl(s_len[b]);
                } while (len == 0);
                n = (len + SK_UNIT - 1) / SK_UNIT;
            }
            seg0 = seg_end;
        }
        return c;
    };

    struct Buf {
        vchunk v[CH][4];
        u32x4_t q[D / 32];
    };
    const int wq = (int)(threadIdx.x >> 6);  // this wave's K slots
    auto kslot = [&](int j) -> uint16_t* {
        return j == 0 ? sK0[wq] : j == 1 ? sK1[wq] : j == 2 ? sK2[wq] : sK3[wq];
    };
    // lane's source offset (bytes, from the chunk's first row) for its i-th
    // K DMA: LDS position p = 64 i + lane holds row p / CPR, logical chunk
    // (p % CPR) ^ (row % CPR)
    uint32_t kvoff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int p = 64 * i + lane, row = p / CPR;
        kvoff[i] = (uint32_t)((row * D + (((p % CPR) ^ (row % CPR)) * 8)) * 2);
    }
    auto load = [&](Buf& f, const Chunk& c, int j) {
        const int cb = rfl(c.b), csg = rfl(c.sg), ck0 = rfl(c.key0), cnk = rfl(c.nk);
        const int kvh = csg / groups, grp = csg % groups;
        const int64_t row0 = ((int64_t)cb * Hkv + kvh) * cap + ck0;
        const uint32_t kbytes = (uint32_t)(cnk * D * 2);
        const buf_rsrc rk = make_rsrc(Kc + row0 * D, kbytes);
        const buf_rsrc rv = make_rsrc(Vc + row0 * D, kbytes);
        const buf_rsrc rq = make_rsrc(Qg + ((int64_t)cb * Hq + kvh * nrep + grp * NR) * D,
                                      cnk ? (uint32_t)(NR * D * 2) : 0u);
#if __HIP_DEVICE_COMPILE__
        constexpr int NT = 2;  // cache policy: non-temporal, the caches are read once
        {
            uint16_t* ks = kslot(j);
#pragma unroll
            for (int i = 0; i < 4; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(ks + 512 * i),
                                                         16, kvoff[i], 0, 0, NT);
        }
#pragma unroll
        for (int kt = 0; kt < CH; kt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t off = (uint32_t)(((16 * kt + 4 * g + r) * D + DL * lq) * 2);
                if constexpr (DL == 8)
                    f.v[kt][r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, NT));
                else
                    f.v[kt][r] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, NT));
            }
        }
#pragma unroll
        for (int cc = 0; cc < D / 32; cc++)
            f.q[cc] = __builtin_amdgcn_raw_buffer_load_b128(rq, (uint32_t)((lq * D + 32 * cc + 8 * g) * 2), 0, 0);
#else
        (void)f;
        (void)rk;
        (void)rv;
        (void)rq;
#endif
    };

    float o[NR][DL];
#pragma unroll
    for (int hh = 0; hh < NR; hh++)
#pragma unroll
        for (int e = 0; e < DL; e++) o[hh][e] = 0.0f;
    float m = -INFINITY, l = 0.0f;  // this lane's head lq; l is the lane's share

    auto compute = [&](const Buf& f, const Chunk& c, int j) {
        f32x4 s[CH];
        const uint16_t* ks = kslot(j);
#pragma unroll
        for (int kt = 0; kt < CH; kt++) {
            s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
            const int row = 16 * kt + lq;
#pragma unroll
            for (int cc = 0; cc < D / 32; cc++) {
                const u32x4_t ka = *reinterpret_cast<const u32x4_t*>(ks + row * D + (((4 * cc + g) ^ (row % CPR)) * 8));
                s[kt] = El<F16>::mfma16(__builtin_bit_cast(typename El<F16>::v8, ka),
                                        __builtin_bit_cast(typename El<F16>::v8, f.q[cc]), s[kt]);
            }
        }
        float t[CH][4];
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < CH; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                t[kt][r] = (16 * kt + 4 * g + r < c.nk) ? s[kt][r] * sl2 : -INFINITY;
                mx = fmaxf(mx, t[kt][r]);
            }
        mx = wave_xor_max(mx);
        const float mn = fmaxf(m, mx);
        const float alpha = (mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
        const float mu = (mn == -INFINITY) ? 0.0f : mn;
        float p[CH][4];
        float ps = 0.0f;
#pragma unroll
        for (int kt = 0; kt < CH; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[kt][r] = __builtin_amdgcn_exp2f(t[kt][r] - mu);
                ps = ps + p[kt][r];
            }
        l = l * alpha + ps;
        m = mn;
#pragma unroll
        for (int hh = 0; hh < NR; hh++) {
            const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), hh));
#pragma unroll
            for (int e = 0; e < DL; e++) o[hh][e] = o[hh][e] * a;
        }
#pragma unroll
        for (int kt = 0; kt < CH; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                uint32_t ws[DL / 2];
                __builtin_memcpy(ws, &f.v[kt][r], sizeof(ws));
                float vf[DL];
#pragma unroll
                for (int e = 0; e < DL / 2; e++) {
                    vf[2 * e] = El<F16>::lo(ws[e]);
                    vf[2 * e + 1] = El<F16>::hi(ws[e]);
                }
#pragma unroll
                for (int hh = 0; hh < NR; hh++) {
                    float pb;
                    switch (hh) {  // lane 16g + hh of this lane's row
                        case 0: pb = dpp_f<0x150>(p[kt][r]); break;
                        case 1: pb = dpp_f<0x151>(p[kt][r]); break;
                        case 2: pb = dpp_f<0x152>(p[kt][r]); break;
                        case 3: pb = dpp_f<0x153>(p[kt][r]); break;
                        case 4: pb = dpp_f<0x154>(p[kt][r]); break;
                        case 5: pb = dpp_f<0x155>(p[kt][r]); break;
                        case 6: pb = dpp_f<0x156>(p[kt][r]); break;
                        default: pb = dpp_f<0x157>(p[kt][r]); break;
                    }
#pragma unroll
                    for (int e = 0; e < DL; e++) o[hh][e] = __builtin_fmaf(pb, vf[e], o[hh][e]);
                }
            }
        if (c.last) {
            const int64_t slot = (int64_t)c.b * G + c.sg + wv;
            const float lt = wave_xor_sum(l);
#pragma unroll
            for (int hh = 0; hh < NR; hh++) {
                float ov[DL];
#pragma unroll
                for (int e = 0; e < DL; e++) ov[e] = wave_xor_sum(o[hh][e]);
                if (g == 0) {
                    float* dst = part_o + (slot * NR + hh) * D + DL * lq;
#pragma unroll
                    for (int e = 0; e < DL; e += 4)
                        *reinterpret_cast<float4*>(dst + e) = make_float4(ov[e], ov[e + 1], ov[e + 2], ov[e + 3]);
                }
            }
            if (g == 0 && lq < NR) part_ml[slot * NR + lq] = make_float2(m, lt);
#pragma unroll
            for (int hh = 0; hh < NR; hh++)
#pragma unroll
                for (int e = 0; e < DL; e++) o[hh][e] = 0.0f;
            m = -INFINITY;
            l = 0.0f;
        }
    };

    // the ring: NB chunks issued up front; each step computes the oldest and
    // refills its slot with the chunk NB ahead, so NB - 1 chunks are in flight
    // while one is computed. The loop is unrolled NB times so that every slot
    // keeps its registers, and no slot is ever free across the loop head
    // (where a register reused as a temporary would make the compiler wait
    // for every load in flight).
    // The first PEEL turns of the ring run as straight-line code: at the loop
    // head the compiler merges the entry and back-edge states and waits for
    // every load in flight, so only waves with more chunks than that reach it.
    Buf f[NB];
    Chunk c[NB];
#pragma unroll
    for (int i = 0; i < NB; i++) {
        c[i] = make();
        load(f[i], c[i], i);
    }
    auto step = [&](int j) {
        if (c[j].nk == 0) return false;
        compute(f[j], c[j], j);
        c[j] = make();
        load(f[j], c[j], j);
        __builtin_amdgcn_sched_barrier(0);
        return true;
    };
    constexpr int PEEL = 3;
#pragma unroll
    for (int t = 0; t < PEEL * NB; t++)
        if (!step(t % NB)) return;
    for (;;) {
#pragma unroll
        for (int j = 0; j < NB; j++)
            if (!step(j)) return;
    }
}

// Merges the stream-K partials of one (sequence, query head) in wave order:
// the waves whose unit ranges meet the segment are those from the wave
// holding its first unit to the wave holding its last (wave of unit u:
// ceil((u+1) W / T) - 1 for ranges [w T / W, (w+1) T / W), with the kernel's
// W = min(grid waves, T), so no wave in between is empty). A sequence with no
// keys gives 0/0, as the split combine does.
template <int D, int NR, typename OT>
__global__ __launch_bounds__(D) void k_decode_sk_combine(const float* __restrict__ part_o,
                                                         const float2* __restrict__ part_ml,
                                                         const int* __restrict__ pref,
                                                         const int32_t* __restrict__ lens, int B, int Hq, int Hkv,
                                                         int nrep, int max_len, int64_t W, OT* __restrict__ out,
                                                         float* __restrict__ lse) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int groups = nrep / NR, G = Hkv * groups;
    const int kvh = h / nrep, hr = h % nrep, grp = hr / NR, hh = hr % NR;
    const int sg = kvh * groups + grp;
    // the sequence's length and the two prefix sums, all three loads in one
    // round trip (as scalar loads the compiler waited for each in turn)
    const buf_rsrc rlen = make_rsrc(lens, (uint32_t)B * 4u), rpre = make_rsrc(pref, (uint32_t)(B + 1) * 4u);
    const float f_len = buf_load_f(rlen, (uint32_t)b * 4u);
    const float f_pb = buf_load_f(rpre, (uint32_t)b * 4u);
    const float f_pT = buf_load_f(rpre, (uint32_t)B * 4u);
    __builtin_amdgcn_sched_barrier(0);
    int len = __builtin_amdgcn_readfirstlane(__float_as_int(f_len));
    len = len < 0 ? 0 : (len > max_len ? max_len : len);
    const int n = (len + SK_UNIT - 1) / SK_UNIT;
    const int64_t T = __builtin_amdgcn_readfirstlane(__float_as_int(f_pT));
    // the kernel's int sums, widened here
    const int64_t u0 = __builtin_amdgcn_readfirstlane(__float_as_int(f_pb)) + (int64_t)sg * n;
    W = W < T ? W : T;
    const int64_t slot0 = (int64_t)b * G + sg;
    float mm = -INFINITY, tl = 0.0f, acc = 0.0f;
    int64_t w_lo = 0, w_hi = -1;
    if (n > 0) {
        // wave of unit u: ceil((u + 1) W / T) - 1 = floor(((u + 1) W - 1) / T)
        w_lo = floordiv_nn((u0 + 1) * W - 1, T);
        w_hi = floordiv_nn((u0 + n) * W - 1, T);
    }
    // batches of CB partials, every load of a batch in flight at once, as
    // unconditional buffer loads (a slot past the segment's last wave reads
    // zero: no memory access, and the compiler counts the loads exactly);
    // the running sums are rescaled when a batch raises the maximum. The
    // first batch (all of them at C4's shapes) is outside the loop, so its
    // waits count only its own loads.
    constexpr int CB = 32;
    const buf_rsrc rml = make_rsrc(part_ml, 0x7fffffffu), ro = make_rsrc(part_o, 0x7fffffffu);
    auto batch = [&](int64_t w0) __attribute__((always_inline)) {
        float2 ml[CB];
        float ov[CB];
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const int64_t sl = (slot0 + w0 + i) * NR + hh;
            const bool on = w0 + i <= w_hi;
            ml[i] = buf_load_f2(rml, on ? (uint32_t)(sl * 8) : BUF_OOB);
            ov[i] = buf_load_f(ro, on ? (uint32_t)((sl * D + d) * 4) : BUF_OOB);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load issued before any result is used
        // absent partials read (0, 0): their m is taken as -inf
#pragma unroll
        for (int i = 0; i < CB; i++)
            if (w0 + i > w_hi) ml[i].x = -INFINITY;
        float bm = mm;
#pragma unroll
        for (int i = 0; i < CB; i++) bm = fmaxf(bm, ml[i].x);
        const float mu = (bm == -INFINITY) ? 0.0f : bm;
        if (mm != -INFINITY) {
            const float a = exp2f(mm - mu);
            tl = tl * a;
            acc = acc * a;
        }
#pragma unroll
        for (int i = 0; i < CB; i++) {
            const float f = exp2f(ml[i].x - mu);  // 0 for the absent entries
            tl = tl + ml[i].y * f;
            acc = acc + ov[i] * f;
        }
        mm = bm;
    };
    if (w_lo <= w_hi) batch(w_lo);
    for (int64_t w0 = w_lo + CB; w0 <= w_hi; w0 += CB) batch(w0);
    const float mu = (mm == -INFINITY) ? 0.0f : mm;
    if constexpr (std::is_same<OT, _Float16>::value)
        reinterpret_cast<uint16_t*>(out)[((int64_t)b * Hq + h) * D + d] = f16_from_f32(acc / tl);
    else if constexpr (sizeof(OT) == 2)
        out[((int64_t)b * Hq + h) * D + d] = bf16_from_f32(acc / tl);
    else
        out[((int64_t)b * Hq + h) * D + d] = acc / tl;
    if (lse && d == 0) lse[(int64_t)b * Hq + h] = mu * LN2 + logf(tl);
}

// Decode, f32 (the precision the reference runs an f32 model in). Grid
// (splits of 256 keys, Hq, B); thread t of a workgroup scores key t of the
// split (a sequential f32 dot over D), the workgroup reduces max and sum,
// then D-wide thread groups accumulate P.V over interleaved keys with
// coalesced V rows and merge in LDS. Writes the same (m, l, O) partial per
// split as the bf16 kernel.
template <int D>
__global__ __launch_bounds__(256) void k_decode_f32(const float* __restrict__ Qg, const float* __restrict__ Kc,
                                                  const float* __restrict__ Vc, int Hq, int Hkv, int nrep, int cap,
                                                  const int32_t* __restrict__ lens, int nsplit, float sl2,
                                                  float* __restrict__ part_o, float2* __restrict__ part_ml) {
    constexpr int G = 256 / D;  // key groups in P.V
    __shared__ __align__(16) float sq[D];
    __shared__ float sp[DEC_SPLIT];
    __shared__ float sred[2][4];
    __shared__ float so[G][D];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / nrep;
    int len = lens[b];
    len = len < 0 ? 0 : (len > cap ? cap : len);
    if (split * DEC_SPLIT >= len) return;  // uniform over the workgroup
    const int k0 = split * DEC_SPLIT;
    const int nk = min(len - k0, DEC_SPLIT);
    const float* kp = Kc + ((int64_t)b * Hkv + kvh) * cap * D;
    const float* vp = Vc + ((int64_t)b * Hkv + kvh) * cap * D;
    if (tid < D) sq[tid] = Qg[((int64_t)b * Hq + h) * D + tid];
    __syncthreads();

    float s = -INFINITY;
    if (tid < nk) {
        const float4* kr = reinterpret_cast<const float4*>(kp + (int64_t)(k0 + tid) * D);
        const float4* qr = reinterpret_cast<const float4*>(sq);
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < D / 4; c++) {
            const float4 kv = kr[c], qv = qr[c];
            acc = acc + qv.x * kv.x;
            acc = acc + qv.y * kv.y;
            acc = acc + qv.z * kv.z;
            acc = acc + qv.w * kv.w;
        }
        s = acc * sl2;
    }
    float mx = s;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) sred[0][w] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(sred[0][0], sred[0][1]), fmaxf(sred[0][2], sred[0][3]));
    const float mu = (m == -INFINITY) ? 0.0f : m;
    const float p = (tid < nk) ? exp2f(s - mu) : 0.0f;
    sp[tid] = p;
    float l = p;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) l = l + __shfl_xor(l, off);
    if (lane == 0) sred[1][w] = l;
    __syncthreads();
    l = (sred[1][0] + sred[1][1]) + (sred[1][2] + sred[1][3]);

    const int d = tid % D, g = tid / D;
    float acc = 0.0f;
    constexpr int U = 8;  // V rows in flight per thread
    for (int t0 = g; t0 < nk; t0 += G * U) {
        float vr[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = t0 + u * G;
            vr[u] = t < nk ? vp[(int64_t)(k0 + t) * D + d] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; u++)
            if (t0 + u * G < nk) acc = acc + sp[t0 + u * G] * vr[u];
    }
    so[g][d] = acc;
    __syncthreads();
    if (tid < D) {
        float o = so[0][tid];
#pragma unroll
        for (int gg = 1; gg < G; gg++) o = o + so[gg][tid];
        const int64_t prow = ((int64_t)b * Hq + h) * nsplit + split;
        part_o[prow * D + tid] = o;
        if (tid == 0) part_ml[prow] = make_float2(m, l);
    }
}

// Decode, f32, single pass: one workgroup per (query head, sequence) over the
// whole sequence, for caches of at most DEC1_MAX_KEYS keys -- the decode
// step's regime, where split partials and a combine launch cost more than
// they save. D/4 lanes share a key row, a float4 each, so every load
// instruction reads whole rows; each lane keeps DEC1_U rows in flight; the
// scores stay in LDS. The first batch of V rows is loaded before the softmax.
constexpr int DEC1_MAX_KEYS = 1024;
constexpr int DEC1_U = 16;

// s_waitcnt lgkmcnt(0) then s_barrier: orders LDS only, global loads stay in flight
__device__ inline void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int D>
__global__ __launch_bounds__(256) void k_decode1_f32(const float* __restrict__ Qg, const float* __restrict__ Kc,
                                                   const float* __restrict__ Vc, int Hq, int Hkv, int nrep, int cap,
                                                   const int32_t* __restrict__ lens, int max_len, float sl2,
                                                   float* __restrict__ out, float* __restrict__ lse) {
    constexpr int TPK = D / 4;     // lanes per key row
    constexpr int RPI = 256 / TPK;  // rows per workgroup per load instruction
    __shared__ float sp[DEC1_MAX_KEYS];
    __shared__ float sred[2][4];
    __shared__ float4 so[4][TPK];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = tid % TPK, kl = tid / TPK;  // float4 of the row, row slot
    const int h = blockIdx.x, b = blockIdx.y, kvh = h / nrep;
    int len = lens[b];
    len = len < 0 ? 0 : (len > max_len ? max_len : len);  // max_len <= min(cap, DEC1_MAX_KEYS)
    const float4* kp = reinterpret_cast<const float4*>(Kc + ((int64_t)b * Hkv + kvh) * cap * D);
    const float4* vp = reinterpret_cast<const float4*>(Vc + ((int64_t)b * Hkv + kvh) * cap * D);
    const float4 qv = reinterpret_cast<const float4*>(Qg + ((int64_t)b * Hq + h) * D)[c];
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);

    float4 rv[DEC1_U];
    auto load_rows = [&](const float4* base, int t0) {
#pragma unroll
        for (int u = 0; u < DEC1_U; u++) {
            const int t = t0 + u * RPI + kl;
            rv[u] = t < len ? base[(int64_t)t * TPK + c] : zero;
        }
    };

    // scores, scaled to log2 units, into LDS
    float mx = -INFINITY;
    for (int t0 = 0; t0 < len; t0 += RPI * DEC1_U) {
        load_rows(kp, t0);
#pragma unroll
        for (int u = 0; u < DEC1_U; u++) {
            float s = qv.x * rv[u].x;
            s = s + qv.y * rv[u].y;
            s = s + qv.z * rv[u].z;
            s = s + qv.w * rv[u].w;
            s = row16_sum(s);
            if constexpr (TPK == 32) s = xor16_sum(s);
            const int t = t0 + u * RPI + kl;
            if (t < len) {
                s = s * sl2;
                mx = fmaxf(mx, s);
                if (c == 0) sp[t] = s;
            }
        }
    }
    load_rows(vp, 0);  // the first V rows travel during the softmax
    mx = wave_xor_max(row16_max(mx));
    if (lane == 0) sred[0][w] = mx;
    lds_barrier();
    const float m = fmaxf(fmaxf(sred[0][0], sred[0][1]), fmaxf(sred[0][2], sred[0][3]));
    const float mu = (m == -INFINITY) ? 0.0f : m;
    float l = 0.0f;
    for (int t = tid; t < len; t += 256) {
        const float p = exp2f(sp[t] - mu);
        sp[t] = p;
        l = l + p;
    }
    l = wave_xor_sum(row16_sum(l));
    if (lane == 0) sred[1][w] = l;
    lds_barrier();
    l = (sred[1][0] + sred[1][1]) + (sred[1][2] + sred[1][3]);

    // P.V: the same row slots; each lane sums its float4 over its rows in order
    float4 acc = zero;
    for (int t0 = 0; t0 < len; t0 += RPI * DEC1_U) {
        if (t0 > 0) load_rows(vp, t0);
#pragma unroll
        for (int u = 0; u < DEC1_U; u++) {
            const int t = t0 + u * RPI + kl;
            if (t < len) {
                const float p = sp[t];
                acc.x = acc.x + p * rv[u].x;
                acc.y = acc.y + p * rv[u].y;
                acc.z = acc.z + p * rv[u].z;
                acc.w = acc.w + p * rv[u].w;
            }
        }
    }
    // the wave's row slots (lanes c, c + TPK, ...), then the four waves
    if constexpr (TPK == 16) {
        acc.x = xor16_sum(acc.x);
        acc.y = xor16_sum(acc.y);
        acc.z = xor16_sum(acc.z);
        acc.w = xor16_sum(acc.w);
    }
    acc.x = xor32_sum(acc.x);
    acc.y = xor32_sum(acc.y);
    acc.z = xor32_sum(acc.z);
    acc.w = xor32_sum(acc.w);
    if (lane < TPK) so[w][lane] = acc;
    lds_barrier();
    if (tid < TPK) {
        float4 o = so[0][tid];
#pragma unroll
        for (int ww = 1; ww < 4; ww++) {
            o.x = o.x + so[ww][tid].x;
            o.y = o.y + so[ww][tid].y;
            o.z = o.z + so[ww][tid].z;
            o.w = o.w + so[ww][tid].w;
        }
        reinterpret_cast<float4*>(out + ((int64_t)b * Hq + h) * D)[tid] =
            make_float4(o.x / l, o.y / l, o.z / l, o.w / l);
        if (lse && tid == 0) lse[(int64_t)b * Hq + h] = mu * LN2 + logf(l);
    }
}

template <int D, typename OT>
__global__ __launch_bounds__(D) void k_decode_combine(const float* __restrict__ part_o,
                                                    const float2* __restrict__ part_ml,
                                                    const int32_t* __restrict__ lens, int Hq, int cap, int nsplit,
                                                    OT* __restrict__ out, float* __restrict__ lse) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int64_t base = ((int64_t)b * Hq + h) * nsplit;
    // the first CMAX splits' partials are requested before the length is
    // known (one round trip for both); splits past it are not used
    constexpr int CMAX = 16;
    float2 mlv[CMAX];
    float pv[CMAX];
#pragma unroll
    for (int s = 0; s < CMAX; s++) {
        if (s < nsplit) {
            mlv[s] = part_ml[base + s];
            pv[s] = part_o[(base + s) * D + d];
        }
    }
    int len = lens[b];
    len = len < 0 ? 0 : (len > cap ? cap : len);
    int ns = (len + DEC_SPLIT - 1) / DEC_SPLIT;
    ns = ns < nsplit ? ns : nsplit;  // a length above max_len is truncated, never read past
    float mm = -INFINITY;
#pragma unroll
    for (int s = 0; s < CMAX; s++)
        if (s < ns) mm = fmaxf(mm, mlv[s].x);
    for (int s = CMAX; s < ns; s++) mm = fmaxf(mm, part_ml[base + s].x);
    const float mu = (mm == -INFINITY) ? 0.0f : mm;
    float tl = 0.0f, acc = 0.0f;
#pragma unroll
    for (int s = 0; s < CMAX; s++) {
        if (s < ns) {
            const float f = exp2f(mlv[s].x - mu);
            tl = tl + mlv[s].y * f;
            acc = acc + pv[s] * f;
        }
    }
    for (int s = CMAX; s < ns; s++) {
        const float2 ml = part_ml[base + s];
        const float f = exp2f(ml.x - mu);
        tl = tl + ml.y * f;
        acc = acc + part_o[(base + s) * D + d] * f;
    }
    if constexpr (std::is_same<OT, _Float16>::value)
        reinterpret_cast<uint16_t*>(out)[((int64_t)b * Hq + h) * D + d] = f16_from_f32(acc / tl);
    else if constexpr (sizeof(OT) == 2)
        out[((int64_t)b * Hq + h) * D + d] = bf16_from_f32(acc / tl);
    else
        out[((int64_t)b * Hq + h) * D + d] = acc / tl;
    if (lse && d == 0) lse[(int64_t)b * Hq + h] = mu * LN2 + logf(tl);
}

const char* OP = "aten._scaled_dot_product_flash_attention_for_cpu.default";

}  // namespace

// Where a decode attention call gets its work buffer (partials, prefix sums):
// the stream's workspace, or the fixed device array of the no-alloc entry.
using ScratchFn = tn_status (*)(hipStream_t, size_t, void**);

// The no-alloc entry's work buffer: one array per GPU, in the code object's
// device memory, held until the process ends. Host code never passes the
// symbol itself (in host code it is a stand-in, not a device address): its
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and is kept per device.
constexpr size_t DECODE_SCRATCH_BYTES = TN_DECODE_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[DECODE_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
std::map<int, void*> g_scratch_addr;

tn_status static_scratch(hipStream_t, size_t bytes, void** out) {
    if (bytes > DECODE_SCRATCH_BYTES) {
        char buf[256];
        std::snprintf(buf, sizeof buf,
                      "tn_sdpa_decode_noalloc: this call needs %zu bytes of work buffer, more than the %zu bytes of "
                      "the fixed device array; use tn_sdpa_decode",
                      bytes, DECODE_SCRATCH_BYTES);
        return fail(TN_EVALUE, buf);
    }
    int dev = 0;
    TN_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch_addr.find(dev);
    if (it == g_scratch_addr.end()) {
        void* p = nullptr;
        TN_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        it = g_scratch_addr.emplace(dev, p).first;
    }
    *out = it->second;
    return TN_OK;
}
}  // namespace

// Argument checks of the decode attention (shared with the decode step).
tn_status decode_check(int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, int64_t max_len) {
    if (dtype != TN_BF16 && dtype != TN_F32 && dtype != TN_F16)
        return fail(TN_ENOTIMPL,
                    "sdpa_decode: only float32, bfloat16 and float16 KV caches are implemented on the hip device");
    if (B < 0 || Hq < 0 || Hkv <= 0 || cap <= 0 || D <= 0 || max_len < 1 || max_len > cap)
        return fail(TN_EINVAL, "sdpa_decode: need Hkv > 0, cap > 0 and 1 <= max_len <= cap");
    if (Hq % Hkv != 0) {
        char buf[256];
        std::snprintf(buf, sizeof buf,
                      "sdpa_decode: grouped-query attention with %lld query heads and %lld key/value heads -- the "
                      "head counts do not divide",
                      (long long)Hq, (long long)Hkv);
        return fail(TN_ENOTIMPL, buf);
    }
    if (D > ANY_DMAX) {
        char buf[256];
        std::snprintf(buf, sizeof buf,
                      "sdpa_decode: head_dim %lld is not implemented on the hip device (kernels exist up to 256)",
                      (long long)D);
        return fail(TN_ENOTIMPL, buf);
    }
    if (B > 65535 || Hq > 65535 || cap > INT32_MAX) return fail(TN_EVALUE, "sdpa_decode: shape too large");
    return TN_OK;
}

// Split-KV decode attention with caller-provided partial buffers (B*Hq*
// ceil(max_len/256) rows of D floats, and as many (m, l) pairs): the grid is
// sized by max_len, each workgroup reads its sequence's length on the device,
// so the launch stays valid for every length up to max_len.
tn_status decode_launch(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, const int32_t* lens,
                        int64_t max_len, double scale, void* out, float* lse, float* part_o, float2* part_ml) {
    const int nrep = (int)(Hq / Hkv);
    const int nsplit = (int)cdiv(max_len, DEC_SPLIT);
    const double sc = std::isnan(scale) ? 1.0 / std::sqrt((double)D) : scale;
    const float sl2 = (float)sc * LOG2E;
    if (D != 64 && D != 128) {
        // the split kernels below exist for head dims 64 and 128; any other
        // (up to 256, decode_check) runs on the plain kernel, one query row per
        // (sequence, head) over the cache's cap rows, as tn_sdpa_decode does
        const dim3 grid(1u, (unsigned)Hq, (unsigned)B);
        if (dtype == TN_F32)
            hipLaunchKernelGGL((k_attn_any<0, 0>), grid, dim3(256), 0, st, q, k_cache, v_cache, (int)Hq, (int)Hkv, 1,
                               (int)cap, (int)D, sc, 0, out, lse, MaskRef{}, lens, (int)max_len);
        else if (dtype == TN_BF16)
            hipLaunchKernelGGL((k_attn_any<1, 0>), grid, dim3(256), 0, st, q, k_cache, v_cache, (int)Hq, (int)Hkv, 1,
                               (int)cap, (int)D, sc, 0, out, lse, MaskRef{}, lens, (int)max_len);
        else
            hipLaunchKernelGGL((k_attn_any<2, 0>), grid, dim3(256), 0, st, q, k_cache, v_cache, (int)Hq, (int)Hkv, 1,
                               (int)cap, (int)D, sc, 0, out, lse, MaskRef{}, lens, (int)max_len);
        TN_LAUNCHED();
        return TN_OK;
    }
    if (dtype == TN_F32) {
        auto qq = static_cast<const float*>(q);
        auto kk = static_cast<const float*>(k_cache);
        auto vv = static_cast<const float*>(v_cache);
        auto oo = static_cast<float*>(out);
        if (max_len <= DEC1_MAX_KEYS) {
            const dim3 g1((unsigned)Hq, (unsigned)B);
            if (D == 128)
                hipLaunchKernelGGL(k_decode1_f32<128>, g1, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, nrep,
                                   (int)cap, lens, (int)max_len, sl2, oo, lse);
            else
                hipLaunchKernelGGL(k_decode1_f32<64>, g1, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, nrep,
                                   (int)cap, lens, (int)max_len, sl2, oo, lse);
            TN_LAUNCHED();
            return TN_OK;
        }
        const dim3 grid((unsigned)nsplit, (unsigned)Hq, (unsigned)B);
        if (D == 128)
            hipLaunchKernelGGL(k_decode_f32<128>, grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, nrep,
                               (int)cap, lens, nsplit, sl2, part_o, part_ml);
        else
            hipLaunchKernelGGL(k_decode_f32<64>, grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, nrep,
                               (int)cap, lens, nsplit, sl2, part_o, part_ml);
        TN_LAUNCHED();
        if (D == 128)
            hipLaunchKernelGGL((k_decode_combine<128, float>), dim3((unsigned)Hq, (unsigned)B), dim3(128), 0, st,
                               part_o, part_ml, lens, (int)Hq, (int)cap, nsplit, oo, lse);
        else
            hipLaunchKernelGGL((k_decode_combine<64, float>), dim3((unsigned)Hq, (unsigned)B), dim3(64), 0, st,
                               part_o, part_ml, lens, (int)Hq, (int)cap, nsplit, oo, lse);
        TN_LAUNCHED();
        return TN_OK;
    }
    // query heads per workgroup: the largest of 8, 4, 3, 2, 1 that divides the group
    const int nr = nrep % 8 == 0 ? 8 : nrep % 4 == 0 ? 4 : nrep % 3 == 0 ? 3 : nrep % 2 == 0 ? 2 : 1;
    auto qq = static_cast<const uint16_t*>(q);
    auto kk = static_cast<const uint16_t*>(k_cache);
    auto vv = static_cast<const uint16_t*>(v_cache);
    dim3 grid((unsigned)nsplit, (unsigned)(Hkv * (nrep / nr)), (unsigned)B);
    const bool h16 = dtype == TN_F16;
#define TN_DEC(DD, NR)                                                                                            \
    do {                                                                                                          \
        if (h16)                                                                                                  \
            hipLaunchKernelGGL((k_decode_bf16<DD, NR, true>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq,       \
                               (int)Hkv, nrep, (int)cap, lens, nsplit, sl2, part_o, part_ml);                     \
        else                                                                                                      \
            hipLaunchKernelGGL((k_decode_bf16<DD, NR>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv,   \
                               nrep, (int)cap, lens, nsplit, sl2, part_o, part_ml);                               \
    } while (0)
#define TN_DEC_D(DD)                       \
    switch (nr) {                          \
        case 8: TN_DEC(DD, 8); break;      \
        case 4: TN_DEC(DD, 4); break;      \
        case 3: TN_DEC(DD, 3); break;      \
        case 2: TN_DEC(DD, 2); break;      \
        default: TN_DEC(DD, 1); break;     \
    }
    if (D == 128) {
        TN_DEC_D(128)
    } else {
        TN_DEC_D(64)
    }
#undef TN_DEC_D
#undef TN_DEC
    TN_LAUNCHED();
    auto oo = static_cast<uint16_t*>(out);
    auto oh = static_cast<_Float16*>(out);
    if (D == 128) {
        if (h16)
            hipLaunchKernelGGL((k_decode_combine<128, _Float16>), dim3((unsigned)Hq, (unsigned)B), dim3(128), 0, st,
                               part_o, part_ml, lens, (int)Hq, (int)cap, nsplit, oh, lse);
        else
            hipLaunchKernelGGL((k_decode_combine<128, uint16_t>), dim3((unsigned)Hq, (unsigned)B), dim3(128), 0, st,
                               part_o, part_ml, lens, (int)Hq, (int)cap, nsplit, oo, lse);
    } else {
        if (h16)
            hipLaunchKernelGGL((k_decode_combine<64, _Float16>), dim3((unsigned)Hq, (unsigned)B), dim3(64), 0, st,
                               part_o, part_ml, lens, (int)Hq, (int)cap, nsplit, oh, lse);
        else
            hipLaunchKernelGGL((k_decode_combine<64, uint16_t>), dim3((unsigned)Hq, (unsigned)B), dim3(64), 0, st,
                               part_o, part_ml, lens, (int)Hq, (int)cap, nsplit, oo, lse);
    }
    TN_LAUNCHED();
    return TN_OK;
}

namespace {

// The stream-K bf16 decode (k_decode_sk_bf16 + k_decode_sk_combine) for
// B <= SK_MAXB, its partials, unit prefix sums and the grid in the stream's
// workspace.
template <int D, int NR, bool F16>
tn_status decode_sk_run(hipStream_t st, const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t B,
                        int64_t Hq, int64_t Hkv, int64_t cap, const int32_t* lens, int64_t max_len, float sl2,
                        uint16_t* out, float* lse, ScratchFn get) {
    const int nrep = (int)(Hq / Hkv);
    const int64_t G = Hkv * (nrep / NR);
    int wgs = 0;
    TN_TRY(resident_workgroups(reinterpret_cast<const void*>(&k_decode_sk_bf16<D, NR, F16>), 256, 0, &wgs));
    const int64_t W = (int64_t)wgs * 4;
    const int64_t slots = B * G + W;
    const size_t po = (size_t)slots * NR * D * sizeof(float);
    const size_t pm = (size_t)slots * NR * sizeof(float2);
    const size_t pp = (size_t)(B + 1) * sizeof(int);
    void* ws = nullptr;
    TN_TRY(get(st, po + pm + pp, &ws));
    float* part_o = static_cast<float*>(ws);
    float2* part_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + po);
    int* pref = reinterpret_cast<int*>(static_cast<char*>(ws) + po + pm);
    hipLaunchKernelGGL((k_decode_sk_bf16<D, NR, F16>), dim3((unsigned)wgs), dim3(256), 0, st, q, kc, vc, (int)B,
                       (int)Hq, (int)Hkv, nrep, (int)cap, lens, (int)max_len, sl2, part_o, part_ml, pref);
    TN_LAUNCHED();
    using OT = typename std::conditional<F16, _Float16, uint16_t>::type;
    hipLaunchKernelGGL((k_decode_sk_combine<D, NR, OT>), dim3((unsigned)Hq, (unsigned)B), dim3(D), 0, st,
                       part_o, part_ml, pref, lens, (int)B, (int)Hq, (int)Hkv, nrep, (int)max_len, W,
                       reinterpret_cast<OT*>(out), lse);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status decode_sk_launch(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, const int32_t* lens,
                           int64_t max_len, double scale, void* out, float* lse, ScratchFn get) {
    const bool h16 = dtype == TN_F16;
    const int nrep = (int)(Hq / Hkv);
    const int nr = nrep % 8 == 0 ? 8 : nrep % 4 == 0 ? 4 : nrep % 3 == 0 ? 3 : nrep % 2 == 0 ? 2 : 1;
    const double sc = std::isnan(scale) ? 1.0 / std::sqrt((double)D) : scale;
    const float sl2 = (float)sc * LOG2E;
    auto qq = static_cast<const uint16_t*>(q);
    auto kk = static_cast<const uint16_t*>(k_cache);
    auto vv = static_cast<const uint16_t*>(v_cache);
    auto oo = static_cast<uint16_t*>(out);
#define TN_SK(DD, NR)                                                                                          \
    return h16 ? decode_sk_run<DD, NR, true>(st, qq, kk, vv, B, Hq, Hkv, cap, lens, max_len, sl2, oo, lse, get) \
               : decode_sk_run<DD, NR, false>(st, qq, kk, vv, B, Hq, Hkv, cap, lens, max_len, sl2, oo, lse, get)
#define TN_SK_D(DD)                    \
    switch (nr) {                      \
        case 8: TN_SK(DD, 8);          \
        case 4: TN_SK(DD, 4);          \
        case 3: TN_SK(DD, 3);          \
        case 2: TN_SK(DD, 2);          \
        default: TN_SK(DD, 1);         \
    }
    if (D == 128) {
        TN_SK_D(128)
    }
    TN_SK_D(64)
#undef TN_SK_D
#undef TN_SK
}

tn_status refuse_head_dim(int64_t D) {
    char buf[256];
    std::snprintf(buf, sizeof buf,
                  "%s: head_dim %lld is not implemented on the hip device (kernels exist up to 256)", OP,
                  (long long)D);
    return fail(TN_ENOTIMPL, buf);
}

// Work list of the bf16 prefill (see FlashWork). Items aim at the tiles of
// the whole call spread over the device's resident workgroups (two per CU),
// at least 16 tiles (1024 keys) each: a split row costs its items a
// published partial, a ticket and a merge at the end (about 4 us on gfx950),
// so rows that fit stay whole. Timestamp sweeps of config 2 over items of
// 8..32 tiles found 16-24 within a few percent of each other and 8 or 32
// clearly slower. Returns the number of workgroups; `nsplit` gets the largest
// split count (the partial layout's stride) and `table` the classes.
int64_t flash_work(int64_t B, int64_t Hq, int64_t L, int64_t S, int causal, int slots, FlashWork& w, int& nsplit,
                   std::vector<uint32_t>& table) {
    const int64_t nqb = cdiv(L, F3_BQ);
    auto ntiles = [&](int64_t qt) {
        return (int)cdiv(causal ? std::min<int64_t>(S, (qt + 1) * F3_BQ) : S, F3_BK);
    };
    int row_max = 0;
    int64_t total = 0;  // tiles of one head
    for (int64_t qt = 0; qt < nqb; qt++) {
        row_max = std::max(row_max, ntiles(qt));
        total += ntiles(qt);
    }
    w.bh = (int)(B * Hq);
    int target = (int)std::min<int64_t>(row_max, std::max<int64_t>(16, cdiv(total * B * Hq, slots)));
    std::vector<std::pair<int, uint32_t>> cls;  // (tiles, qt | split << 16)
    for (;;) {
        cls.clear();
        for (int64_t qt = nqb - 1; qt >= 0 && (int64_t)cls.size() <= FLASH_MAX_CLS; qt--) {
            const int n = ntiles(qt), ns = row_splits(n, target);
            for (int sp = 0; sp < ns; sp++)
                cls.emplace_back((sp + 1) * n / ns - sp * n / ns, (uint32_t)qt | ((uint32_t)sp << 16));
        }
        if (target >= row_max || (int64_t)cls.size() <= FLASH_MAX_CLS) break;
        target = std::min(row_max, target * 2);  // too many classes for the table: coarser items
    }
    w.target = target;
    if (target >= row_max) {  // nothing split: class c is query block nqb-1-c
        w.ncls = 0;
        nsplit = 1;
        return nqb * B * Hq;
    }
    // longest first: the dispatcher hands out workgroups in order, and
    // consecutive workgroups go to different XCDs
    std::stable_sort(cls.begin(), cls.end(), [](const auto& a, const auto& b) { return a.first > b.first; });
    w.ncls = (int)cls.size();
    nsplit = 1;
    table.resize(cls.size());
    for (size_t i = 0; i < cls.size(); i++) {
        table[i] = cls[i].second;
        nsplit = std::max(nsplit, (int)(cls[i].second >> 16) + 1);
    }
    return (int64_t)w.ncls * B * Hq;
}

// The work list of a shape, built once and kept in device memory for the
// life of the process (a few KB per distinct (device, B*Hq, L, S, causal)):
// the kernel reads its class with one scalar load, and a launch passes a
// pointer instead of the table.
struct PlanKey {
    int dev;
    int64_t bh, L, S;
    int causal, D;
    bool operator<(const PlanKey& o) const {
        return std::tie(dev, bh, L, S, causal, D) < std::tie(o.dev, o.bh, o.L, o.S, o.causal, o.D);
    }
};
struct Plan {
    FlashWork w;
    int nsplit;
    int64_t nitems;
};
std::mutex g_plan_mu;
std::map<PlanKey, Plan> g_plans;

tn_status flash_plan(hipStream_t st, int64_t B, int64_t Hq, int64_t L, int64_t S, int causal, int D, int slots,
                     Plan& out) {
    int dev = 0;
    TN_HIP(hipGetDevice(&dev));
    const PlanKey key{dev, B * Hq, L, S, causal, D};
    std::lock_guard<std::mutex> lock(g_plan_mu);
    auto it = g_plans.find(key);
    if (it != g_plans.end()) {
        out = it->second;
        return TN_OK;
    }
    Plan p{};
    std::vector<uint32_t> table;
    p.nitems = flash_work(B, Hq, L, S, causal, slots, p.w, p.nsplit, table);
    p.w.cls = nullptr;
    if (!table.empty() && table.size() <= (size_t)FLASH_INLINE) {
        std::copy(table.begin(), table.end(), p.w.inl);
    } else if (!table.empty()) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        TN_HIP(hipStreamIsCapturing(st, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return fail(TN_EINVAL, std::string(OP) + ": the first call of a shape cannot be captured (its work list "
                                                     "is uploaded then); make one call before capturing");
        uint32_t* d = nullptr;
        TN_HIP(hipMalloc(reinterpret_cast<void**>(&d), table.size() * sizeof(uint32_t)));
        const hipError_t e = hipMemcpy(d, table.data(), table.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return hip_fail(e, "hipMemcpy (prefill work list)");
        }
        p.w.cls = d;
    }
    g_plans[key] = p;
    out = p;
    return TN_OK;
}

}  // namespace
}  // namespace tn

using namespace tn;

extern "C" {

tn_status tn_sdpa_fwd(void* stream, int dtype, const void* q, const void* k, const void* v, int64_t B, int64_t Hq,
                      int64_t Hkv, int64_t L, int64_t S, int64_t D, const void* attn_mask, int mask_dtype,
                      const int64_t* mask_strides, int is_causal, double scale, void* out, float* lse) {
    if (dtype != TN_F32 && dtype != TN_BF16 && dtype != TN_F16 && dtype != TN_F64)
        return fail(TN_EINVAL, "scaled_dot_product_attention_flash_attention: Expected data type in FP32, FP64, BF16, "
                               "FP16");
    if (B < 0 || Hq < 0 || L < 0 || S < 0 || D < 0 || Hkv < 0)
        return fail(TN_EINVAL, std::string(OP) + ": negative dimension");
    if (D == 0 || S == 0) {
        char buf[256];
        std::snprintf(buf, sizeof buf,
                      "%s: a zero key length or head dimension (query [%lld, %lld, %lld, %lld], key [%lld, %lld, "
                      "%lld, %lld]) is not implemented in torch._C shim",
                      OP, (long long)B, (long long)Hq, (long long)L, (long long)D, (long long)B, (long long)Hkv,
                      (long long)S, (long long)D);
        return fail(TN_ENOTIMPL, buf);
    }
    if (Hkv == 0 || Hq % Hkv != 0) {
        char buf[384];
        std::snprintf(buf, sizeof buf,
                      "%s: grouped-query attention with %lld query heads and %lld key/value heads is not implemented "
                      "in torch._C shim -- the head counts do not divide",
                      OP, (long long)Hq, (long long)Hkv);
        return fail(TN_ENOTIMPL, buf);
    }
    // the mask is the query's dtype or float32 (aten.rs:10142-10150), or a
    // bool one, read as F.sdpa's where(mask, 0, -inf) in the query's dtype
    if (attn_mask && mask_dtype != dtype && mask_dtype != TN_F32 && mask_dtype != TN_BOOL)
        return fail(TN_EINVAL, "scaled_dot_product_attention_flash_attention: Attention mask is the same data type "
                               "as query");
    // an f64 query with an f32 mask is refused by name (aten.rs:10160-10170)
    if (attn_mask && dtype == TN_F64 && mask_dtype == TN_F32)
        return fail(TN_ENOTIMPL, "aten._scaled_dot_product_flash_attention_for_cpu: a float32 attn_mask on a float64 "
                                 "query is refused. Pass the mask as float64.");
    // 0 none, 1 f32, 2 the query's dtype, 3 bool: the kernels' MASK parameter
    const int mk = !attn_mask ? 0 : mask_dtype == TN_F32 ? 1 : mask_dtype == TN_BOOL ? 3 : 2;
    // element strides over (B, Hq, L, S); null: dense [B, Hq, L, S]
    MaskRef mref{attn_mask, Hq * L * S, L * S, S, 1};
    if (attn_mask && mask_strides) {
        for (int i = 0; i < 4; i++)
            if (mask_strides[i] < 0)
                return fail(TN_EVALUE, std::string(OP) + ": attn_mask strides must be non-negative");
        mref.sb = mask_strides[0];
        mref.sh = mask_strides[1];
        mref.sl = mask_strides[2];
        mref.sk = mask_strides[3];
    }
    if (D > ANY_DMAX) return refuse_head_dim(D);
    if (B * Hq * L == 0) return TN_OK;  // nothing to write (aten.rs:10242-10259 returns empty zeros)
    if (!q || !k || !v || !out) return fail(TN_EVALUE, std::string(OP) + ": null pointer");
    if (L > INT32_MAX || S > INT32_MAX || Hq > 65535 || B > 65535)
        return fail(TN_EVALUE, std::string(OP) + ": shape too large");
    const double sc = std::isnan(scale) ? 1.0 / std::sqrt((double)D) : scale;
    const float sl2 = (float)sc * LOG2E;
    hipStream_t st = (hipStream_t)stream;
    const int c = is_causal ? 1 : 0;
    const int64_t rows = B * Hq * L;
    // the MFMA kernels take the row maximum of the unscaled scores (right for
    // scale >= 0) and exist for head dims 64 and 128; anything else runs on
    // the plain kernel
    if ((D != 64 && D != 128) || sc < 0.0 || dtype == TN_F64) {
        const dim3 grid((unsigned)cdiv(L, ANY_BQ), (unsigned)Hq, (unsigned)B);
        const int et = dtype == TN_F32 ? 0 : dtype == TN_BF16 ? 1 : dtype == TN_F16 ? 2 : 3;
#define TN_ANY(ET, MK)                                                                                            \
    hipLaunchKernelGGL((k_attn_any<ET, MK>), grid, dim3(256), 0, st, q, k, v, (int)Hq, (int)Hkv, (int)L, (int)S, \
                       (int)D, sc, c, out, lse, mref, nullptr, 0)
#define TN_ANY_MK(ET)                     \
    do {                                  \
        if (mk == 0) TN_ANY(ET, 0);       \
        else if (mk == 1) TN_ANY(ET, 1);  \
        else if (mk == 3) TN_ANY(ET, 3);  \
        else TN_ANY(ET, 2);               \
    } while (0)
        if (et == 0) TN_ANY_MK(0);
        else if (et == 1) TN_ANY_MK(1);
        else if (et == 2) TN_ANY_MK(2);
        else TN_ANY_MK(3);
#undef TN_ANY_MK
#undef TN_ANY
        TN_LAUNCHED();
        return TN_OK;
    }
    if (dtype == TN_BF16 || dtype == TN_F16) {
        // the key/value buffer descriptors cover one head's S*D elements
        if (S * D * 2 > INT32_MAX) return fail(TN_EVALUE, std::string(OP) + ": key length too large");
        // Small D=64 work (up to four 64-query blocks per CU, where the
        // split-row kernel below would have to split rows to fill the chip)
        // runs without splits on flash64.hip, unmasked or with a mask that is
        // the same for every query row (a key padding mask, [B, 1, 1, S]);
        // larger work keeps the split-row kernel, which is faster once every
        // CU has several blocks.
        if (D == 64 && (mk == 0 || mref.sl == 0) && B * Hq * cdiv(L, 64) <= 1024)
            return flash64_launch(st, dtype == TN_F16, mk, attn_mask, mref.sb, mref.sh, mref.sl, mref.sk,
                                  static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                  static_cast<const uint16_t*>(v), B, Hq, Hkv, L, S, sl2, c,
                                  static_cast<uint16_t*>(out), lse);
        // resident workgroups of the prefill kernel: the slots the schedule is planned over
        int slots = 0;
        tn_status sp = resident_workgroups(D == 64 ? reinterpret_cast<const void*>(&k_flash16<64>)
                                                    : reinterpret_cast<const void*>(&k_flash16<128>),
                                           128 * FlashCfg<64>::KG, 0, &slots);
        if (sp != TN_OK) return sp;
        Plan plan;
        sp = flash_plan(st, B, Hq, L, S, c, (int)D, std::max(slots, 1), plan);
        if (sp != TN_OK) return sp;
        const FlashWork work = plan.w;
        const int nsplit = plan.nsplit;
        const int64_t nitems = plan.nitems;
        if (nitems > INT32_MAX) return fail(TN_EVALUE, std::string(OP) + ": shape too large");
        float* part_o = nullptr;
        float2* part_ml = nullptr;
        uint32_t* tick = nullptr;
        if (nsplit > 1) {
            const size_t po = (size_t)rows * nsplit * D * sizeof(float);
            const size_t pm = (size_t)rows * nsplit * sizeof(float2);
            if ((size_t)F3_BQ * nsplit * D * sizeof(float) > UINT32_MAX)
                return fail(TN_EVALUE, std::string(OP) + ": too many splits");
            void* ws = nullptr;
            tn_status s = workspace(st, po + pm, &ws);
            if (s != TN_OK) return s;
            part_o = static_cast<float*>(ws);
            part_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + po);
            // one counter per (batch, head, query block)
            s = tickets(st, (size_t)(B * Hq) * (size_t)cdiv(L, F3_BQ), &tick);
            if (s != TN_OK) return s;
        }
        auto qq = static_cast<const uint16_t*>(q);
        auto kk = static_cast<const uint16_t*>(k);
        auto vv = static_cast<const uint16_t*>(v);
        auto oo = static_cast<uint16_t*>(out);
        // split rows are merged inside the kernel (merge_split_rows)
#define TN_FLASH(DD, MK, H)                                                                                      \
    hipLaunchKernelGGL((k_flash16<DD, MK, H>), dim3((unsigned)nitems), dim3(128 * FlashCfg<DD>::KG), 0, st, qq, kk, \
                       vv, (int)Hq, (int)Hkv, (int)L, (int)S, sl2, c, work, nsplit, oo, lse, part_o, part_ml, tick,   \
                       mref)
#define TN_FLASH_MK(DD, H)              \
    do {                                \
        if (mk == 0) TN_FLASH(DD, 0, H); \
        else if (mk == 1) TN_FLASH(DD, 1, H); \
        else if (mk == 3) TN_FLASH(DD, 3, H); \
        else TN_FLASH(DD, 2, H);        \
    } while (0)
        const bool h16 = dtype == TN_F16;
        if (D == 64) {
            if (h16) TN_FLASH_MK(64, true); else TN_FLASH_MK(64, false);
        } else {
            if (h16) TN_FLASH_MK(128, true); else TN_FLASH_MK(128, false);
        }
#undef TN_FLASH_MK
#undef TN_FLASH
        TN_LAUNCHED();
        return TN_OK;
    }
    const int bk = (D == 128) ? 32 : PF_BK;
    // the stream-K grid: one workgroup per resident slot, at most one per unit
    int slots = 0;
    {
        tn_status sp = resident_workgroups(D == 64 ? reinterpret_cast<const void*>(&k_fa_f32<64, 64, 0>)
                                                    : reinterpret_cast<const void*>(&k_fa_f32<128, 32, 0>),
                                           PF_THREADS, 0, &slots);
        if (sp != TN_OK) return sp;
    }
    SkGeo geo;
    geo.nqb = (int)cdiv(L, PF_BQ);
    geo.NS = (int)cdiv(S, bk);
    geo.c = PF_BQ / bk;
    geo.causal = c;
    geo.Tbh = geo.P(geo.nqb);
    geo.T = B * Hq * geo.Tbh;
    geo.G = std::min<int64_t>(std::max(slots, 1), geo.T);
    float* part_o = nullptr;
    float2* part_ml = nullptr;
    uint32_t* tick = nullptr;
    if (geo.G > 1) {
        const size_t po = (size_t)(2 * geo.G) * PF_BQ * D * sizeof(float);
        const size_t pm = (size_t)(2 * geo.G) * PF_BQ * sizeof(float2);
        void* ws = nullptr;
        tn_status s = workspace(st, po + pm, &ws);
        if (s != TN_OK) return s;
        part_o = static_cast<float*>(ws);
        part_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + po);
        // one counter per (batch, head, query block); only cut blocks take tickets
        s = tickets(st, (size_t)(B * Hq) * (size_t)geo.nqb, &tick);
        if (s != TN_OK) return s;
    }
    {
        auto qq = static_cast<const float*>(q);
        auto kk = static_cast<const float*>(k);
        auto vv = static_cast<const float*>(v);
        auto oo = static_cast<float*>(out);
        // an f32 query takes an f32 mask (mk 1) or a bool one (mk 3)
#define TN_FA(DD, BKK, MK)                                                                                       \
    hipLaunchKernelGGL((k_fa_f32<DD, BKK, MK>), dim3((unsigned)geo.G), dim3(PF_THREADS), 0, st, qq, kk, vv,      \
                       (int)Hq, (int)Hkv, (int)L, (int)S, sl2, c, geo, oo, lse, part_o, part_ml, tick, mref)
        if (D == 64) {
            if (mk == 1) TN_FA(64, 64, 1);
            else if (mk == 3) TN_FA(64, 64, 3);
            else TN_FA(64, 64, 0);
        } else {
            if (mk == 1) TN_FA(128, 32, 1);
            else if (mk == 3) TN_FA(128, 32, 3);
            else TN_FA(128, 32, 0);
        }
#undef TN_FA
        TN_LAUNCHED();
    }
    return TN_OK;
}

}  // extern "C"

namespace {

// tn_sdpa_decode and its no-alloc twin: the same kernels, the work buffer from `get`.
tn_status decode_entry(void* stream, int dtype, const void* q, const void* k_cache, const void* v_cache, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, const int32_t* lens, int64_t max_len,
                       double scale, void* out, float* lse, ScratchFn get) {
    tn_status s = decode_check(dtype, B, Hq, Hkv, cap, D, max_len);
    if (s != TN_OK || B == 0 || Hq == 0) return s;
    if (!q || !k_cache || !v_cache || !out || !lens) return fail(TN_EVALUE, "sdpa_decode: null pointer");
    // the f32 kernels move rows in 16-byte pieces
    if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) % 16 != 0)
        return fail(TN_EINVAL, "sdpa_decode: q, the caches and out must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (D != 64 && D != 128) {
        // the plain kernel: one query row per (sequence, head), the cache's cap
        // rows as its keys, each sequence's length from lens
        const double sc = std::isnan(scale) ? 1.0 / std::sqrt((double)D) : scale;
        const dim3 grid(1u, (unsigned)Hq, (unsigned)B);
        if (dtype == TN_F32)
            hipLaunchKernelGGL((k_attn_any<0, 0>), grid, dim3(256), 0, st, q, k_cache, v_cache, (int)Hq, (int)Hkv, 1,
                               (int)cap, (int)D, sc, 0, out, lse, MaskRef{}, lens, (int)max_len);
        else if (dtype == TN_BF16)
            hipLaunchKernelGGL((k_attn_any<1, 0>), grid, dim3(256), 0, st, q, k_cache, v_cache, (int)Hq, (int)Hkv, 1,
                               (int)cap, (int)D, sc, 0, out, lse, MaskRef{}, lens, (int)max_len);
        else
            hipLaunchKernelGGL((k_attn_any<2, 0>), grid, dim3(256), 0, st, q, k_cache, v_cache, (int)Hq, (int)Hkv, 1,
                               (int)cap, (int)D, sc, 0, out, lse, MaskRef{}, lens, (int)max_len);
        TN_LAUNCHED();
        return TN_OK;
    }
    // the stream-K kernel counts 16-key units of all segments in an int
    const bool half = dtype == TN_BF16 || dtype == TN_F16;
    if (half && B <= SK_MAXB && B * Hq * cdiv(max_len, SK_UNIT) <= INT32_MAX)
        return decode_sk_launch(st, dtype, q, k_cache, v_cache, B, Hq, Hkv, cap, D, lens, max_len, scale, out, lse,
                                get);
    // the split kernel below takes the row maximum before scaling
    if (half && scale < 0.0)
        return fail(TN_ENOTIMPL, "sdpa_decode: a negative scale is not implemented on the hip device for more than 1024 "
                                 "16-bit sequences");
    const int64_t nsplit = cdiv(max_len, DEC_SPLIT);
    const size_t po = (size_t)B * Hq * nsplit * D * sizeof(float);
    const size_t pm = (size_t)B * Hq * nsplit * sizeof(float2);
    // the single-pass f32 kernel takes no partials
    const bool one_pass = dtype == TN_F32 && max_len <= DEC1_MAX_KEYS;
    void* ws = nullptr;
    if (!one_pass) {
        s = get(st, po + pm, &ws);
        if (s != TN_OK) return s;
    }
    float2* part_ml = ws ? reinterpret_cast<float2*>(static_cast<char*>(ws) + po) : nullptr;
    return decode_launch(st, dtype, q, k_cache, v_cache, B, Hq, Hkv, cap, D, lens, max_len, scale, out, lse,
                         static_cast<float*>(ws), part_ml);
}

}  // namespace

extern "C" {

tn_status tn_sdpa_decode(void* stream, int dtype, const void* q, const void* k_cache, const void* v_cache, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, const int32_t* lens, int64_t max_len,
                         double scale, void* out, float* lse) {
    return decode_entry(stream, dtype, q, k_cache, v_cache, B, Hq, Hkv, cap, D, lens, max_len, scale, out, lse,
                        workspace);
}

tn_status tn_sdpa_decode_noalloc(void* stream, int dtype, const void* q, const void* k_cache, const void* v_cache,
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, const int32_t* lens,
                                 int64_t max_len, double scale, void* out, float* lse) {
    return decode_entry(stream, dtype, q, k_cache, v_cache, B, Hq, Hkv, cap, D, lens, max_len, scale, out, lse,
                        static_scratch);
}

}  // extern "C"

// Outlier-pathway backward for gfx950: gradients of causal softmax attention
// with QK width R and value width D.
//
// No reference counterpart in the repository's own code: the reference
// trains through autograd of torch SDPA (src/HybridOutlierFactorizedAttentionTrain.py:258-259).
//
// With P = exp2(c S - lse) (c = sm_scale * log2(e), lse base 2),
// dP = dO V^T, dS = P (.) (dP - Dt), Dt = rowsum(dO (.) O):
//   dV = P^T dO,  dK = sm_scale dS^T Q,  dQ = sm_scale dS K.
// Two kernels, no atomics:
//   attn_bwd_dkdv_kernel  block = 128 keys (4 waves x 32, lane = key), loop over
//                         the 64-query tiles at or after the block; S and dP in
//                         the C[query, key] layout, so P and dS feed the dV^T and
//                         dK^T products straight from registers as B operands.
//   attn_bwd_dq_kernel    block = 128 queries (4 waves x 32, lane = query), loop
//                         over the 64-key tiles up to the diagonal; S^T, dP^T in
//                         the C[key, query] layout, dQ^T = K^T dS^T.
// The key (dK/dV kernel) or query (dQ kernel) operand of the logits carries
// c as a 16-bit hi/lo pair, and the per-query terms -lse and -Dt enter the S
// and dP products as one extra k-step (a hi/lo pair times ones), so the
// accumulators come out of the matrix cores as c S - lse and dP - Dt and the
// softmax needs one exp2 and one multiply per score.
// Q/dO (dK/dV kernel) and K/V (dQ kernel) tiles are staged in LDS row-major
// only; the operands that run along the tile's rows (dO^T, Q^T, K^T) are read
// with gfx950's transposing LDS load ds_read_b64_tr_b16.  Tile rows are
// swizzled in 16-byte granules so the row reads, the transposing reads and the
// staging stores are free of bank conflicts.
// Matrix operands are 16-bit (bf16 for bf16/f32 inputs, f16 for f16) with f32
// accumulation, as in flash-attention backward passes; f32 inputs form the
// logits from hi/lo operand pairs so the recomputed probabilities agree with
// the forward's log-sum-exp.
#include <cmath>
#include <type_traits>

#include "hofa_tile.h"

namespace hofa {
namespace {

using namespace tile;
constexpr int BQ = 64;   // query tile of the dK/dV kernel
constexpr int BKB = 128; // key block of the dK/dV kernel (4 waves x 32)
constexpr int BM = 128;  // query block of the dQ kernel
constexpr int BN = 64;   // key tile of the dQ kernel

struct AttnBwdK {
    const void *q, *k, *v, *dO;
    const float *lse, *dt;
    void *dq, *dk, *dv;
    int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
    int64_t dq_sb, dq_sh, dq_st, dk_sb, dk_sh, dk_st, dv_sb, dv_sh, dv_st;
    int B, H, T;
    int dv_accumulate;
    float c;         // sm_scale * log2(e)
    float sm_scale;
};

// Scheduling hint for the row-operand products: the LDS reads of the block
// issue as one group ahead of its matrix products, so their latencies overlap
// instead of each read being waited for just before its product.
// The logits' products (NS of them) go first so the exp2 of the softmax can
// overlap the dP products that follow.
template <int NS, int NP>
__device__ __forceinline__ void sched_reads_then_mfma() {
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // DS reads
    __builtin_amdgcn_sched_group_barrier(0x008, NS, 0);  // MFMA: S
    __builtin_amdgcn_sched_group_barrier(0x008, NP, 0);  // MFMA: dP
}

// Four consecutive elements of a gradient row (8-byte aligned for 16-bit
// types, 16-byte for f32): one vector load / store, rounding on store.
template <int DT>
struct Run4 {
    using in_t = typename Stor<DT>::type;
    using raw_t = typename std::conditional<DT == HOFA_F32, f32x4, uint2>::type;
    raw_t r;
    __device__ static Run4 load(const in_t *p) { return Run4{*(const raw_t *)p}; }
    __device__ float get(int e) const {
        if constexpr (DT == HOFA_F32) return r[e];
        else return to_f32<DT>((uint16_t)((e < 2 ? r.x : r.y) >> (16 * (e & 1))));
    }
    __device__ static void store(in_t *p, const float *x) {
        if constexpr (DT == HOFA_F32) {
            *(f32x4 *)p = f32x4{x[0], x[1], x[2], x[3]};
        } else {
            *(uint2 *)p = uint2{pack2<DT>(x[0], x[1]), pack2<DT>(x[2], x[3])};
        }
    }
};

template <int DT, int R, int D>
constexpr int dkdv_occupancy() { return (DT != HOFA_F32 && D == 64 && R <= 32) ? 3 : 1; }
template <int DT, int R, int D>
constexpr int dq_occupancy() { return (DT != HOFA_F32 && D == 64 && R <= 32) ? 4 : 1; }

template <int DT, int R, int D>
__global__ __launch_bounds__(NT, (dkdv_occupancy<DT, R, D>())) void attn_bwd_dkdv_kernel(AttnBwdK a) {
    using in_t = typename Stor<DT>::type;
    using LQ = TileL<R>;
    using LO = TileL<D>;
    constexpr int KS = R / 16, DKS = D / 16, MB = D / 32;
    constexpr int RB = (R + 31) / 32;  // 32-row blocks of dK^T
    constexpr bool SPL = DT == HOFA_F32;
    __shared__ __attribute__((aligned(16))) uint16_t sQ[2][LQ::ELEMS];
    __shared__ __attribute__((aligned(16))) uint16_t sQlo[2][SPL ? LQ::ELEMS : 8];
    __shared__ __attribute__((aligned(16))) uint16_t sO[2][LO::ELEMS];
    __shared__ __attribute__((aligned(16))) uint32_t sX[2][2][BQ];  // per query: (-lse/c, -Dt) as hi/lo pairs

    const int nkb = (a.T + BKB - 1) / BKB;
    int bh, kblk;
    xcd_rank_remap(blockIdx.x, nkb, a.B * a.H, &bh, &kblk);  // key blocks near 0 have the most work
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int k0 = kblk * BKB;
    const int kw0 = k0 + 32 * w;
    const int key = kw0 + (lane & 31);

    const in_t *qp = (const in_t *)a.q + b * a.q_sb + h * a.q_sh;
    const in_t *kp = (const in_t *)a.k + b * a.k_sb + h * a.k_sh;
    const in_t *vp = (const in_t *)a.v + b * a.v_sb + h * a.v_sh;
    const in_t *op = (const in_t *)a.dO + b * a.o_sb + h * a.o_sh;
    const float *lse = a.lse + (int64_t)bh * a.T;
    const float *dtp = a.dt + (int64_t)bh * a.T;

    // B operands: c K as a hi/lo pair (k = dims), so the logits come out of the
    // matrix cores in base-2 units, V (k = dv) of this lane's key, and ones
    // for the shift k-step; loaded once the first tile's loads are issued
    u32x4 kh[KS], kl[KS], vop[DKS];
    const u32x4 ones = {hi ? 0u : kOnes2<DT>, 0u, 0u, 0u};

    f32x16 dvt[MB], dkt[RB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) dvt[mb][v] = 0.f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int v = 0; v < 16; ++v) dkt[rb][v] = 0.f;

    TileStage<DT, R> stq;
    TileStage<DT, D> sto;
    TileDma<R> dmq;
    TileDma<D> dmo;
    if constexpr (!SPL) {
        dmq.init(qp, a.q_st, a.T, w, lane);
        dmo.init(op, a.o_st, a.T, w, lane);
    }
    // per-query lse / Dt of the staged tile: raw loads at fetch (no wait on
    // the tile's loads in flight), shifted hi/lo pairs formed at put
    float ls = 0.f, ds = 0.f;
    auto fetch = [&](int buf, int q0) {
        if constexpr (SPL) {
            stq.fetch(qp, a.q_st, q0, a.T);
            sto.fetch(op, a.o_st, q0, a.T);
        } else {
            dmq.fetch(sQ[buf], q0, w);
            dmo.fetch(sO[buf], q0, w);
        }
        if (tid < BQ) {
            const int qi = min(q0 + tid, a.T - 1);
            ls = lse[qi];
            ds = dtp[qi];
        }
    };
    auto put = [&](int buf, int q0) {
        if constexpr (SPL) {
            stq.put(sQ[buf], sQlo[buf]);
            sto.put(sO[buf], nullptr);
        } else {
            wait_vmem();
        }
        if (tid < BQ) {
            const bool in = q0 + tid < a.T;
            sX[buf][0][tid] = split_pair<DT>(in ? -ls : 0.f);
            sX[buf][1][tid] = split_pair<DT>(in ? -ds : 0.f);
        }
    };
    // One 64-query tile from LDS buffer buf.
    auto tile = [&](int buf, int q0) {
        const bool more = q0 + BQ < a.T;
        if (more) fetch(buf ^ 1, q0 + BQ);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int qq0 = q0 + 32 * qb;
            if (qq0 + 31 < kw0) continue;  // every query of the block precedes this wave's keys
            const int rq = 32 * qb + (lane & 31);
            // this block's query rows: every row operand read is issued before the products
            u32x4 qa[KS], qla[SPL ? KS : 1], oa[DKS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                qa[ks] = *(const u32x4 *)&sQ[buf][LQ::off(rq, 16 * ks + 8 * hi)];
                if constexpr (SPL) qla[ks] = *(const u32x4 *)&sQlo[buf][LQ::off(rq, 16 * ks + 8 * hi)];
            }
#pragma unroll
            for (int ks = 0; ks < DKS; ++ks) oa[ks] = *(const u32x4 *)&sO[buf][LO::off(rq, 16 * ks + 8 * hi)];
            const uint32_t x2 = sX[buf][0][rq], y2 = sX[buf][1][rq];
            const u32x4 xa = {hi ? 0u : x2, 0u, 0u, 0u};
            const u32x4 ya = {hi ? 0u : y2, 0u, 0u, 0u};
            // S' = c Q K^T - lse and dP' = dO V^T - Dt in C[query, key]
            f32x16 s = {}, dp = {};
            sched_reads_then_mfma<KS * (SPL ? 3 : 2) + 1, DKS + 1>();
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                s = mfma32<DT>(qa[ks], kh[ks], s);
                s = mfma32<DT>(qa[ks], kl[ks], s);
                if constexpr (SPL) s = mfma32<DT>(qla[ks], kh[ks], s);
            }
            s = mfma32<DT>(xa, ones, s);
#pragma unroll
            for (int ks = 0; ks < DKS; ++ks) dp = mfma32<DT>(oa[ks], vop[ks], dp);
            dp = mfma32<DT>(ya, ones, dp);
            // P and dS in place (lane = key, v -> query 8(v/4) + 4hi + v%4 of the block).
            // Blocks on the diagonal or past T mask their logits to -inf first
            // (query offset qo is visible iff vlo <= qo <= vhi), so P = 0 there.
            if (qq0 < kw0 + 31 || qq0 + 31 >= a.T || kw0 + 31 >= a.T) {
                const int vlo = key - qq0 - 4 * hi;
                const int vhi = key < a.T ? a.T - 1 - qq0 - 4 * hi : vlo - 1;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int qo = 8 * (v / 4) + (v % 4);
                    if ((uint32_t)(qo - vlo) > (uint32_t)(vhi - vlo)) s[v] = -INFINITY;
                }
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float p = fast_exp2(s[v]);
                s[v] = p;
                dp[v] *= p;
            }
            // dV^T += dO^T P and dK^T += Q^T dS, the row-direction operands read transposed
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const u32x4 pb = pack8<DT>(s, 8 * k2);
                const u32x4 db = pack8<DT>(dp, 8 * k2);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    dvt[mb] = mfma32<DT>(tr_operand<D>(sO[buf], 32 * qb + 16 * k2, 32 * mb, lane), pb, dvt[mb]);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
                    dkt[rb] = mfma32<DT>(tr_operand<R>(sQ[buf], 32 * qb + 16 * k2, 32 * rb, lane), db, dkt[rb]);
            }
        }
        if (more) put(buf ^ 1, q0 + BQ);
        __syncthreads();
    };
    fetch(0, k0);
    // this lane's key operands after the first tile's requests (one memory round
    // trip; the raw V rows before K, whose scaling waits for its load)
#pragma unroll
    for (int ks = 0; ks < DKS; ++ks)
        vop[ks] = key < a.T ? load_op8<DT>(vp + (int64_t)key * a.v_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        load_scaled_op8<DT>(kp + (int64_t)key * a.k_st + 16 * ks + 8 * hi, a.c, key < a.T, kh[ks], kl[ks]);
    put(0, k0);
    __syncthreads();
    for (int q0 = k0, buf = 0; q0 < a.T; q0 += BQ, buf ^= 1) tile(buf, q0);
    if (key >= a.T) return;
    // dV^T / dK^T: lane = key, rows 8(v/4) + 4hi + v%4 of each 32-row block,
    // i.e. runs of four consecutive columns of the key's gradient rows
    in_t *dvr = (in_t *)a.dv + b * a.dv_sb + h * a.dv_sh + (int64_t)key * a.dv_st;
    in_t *dkr = (in_t *)a.dk + b * a.dk_sb + h * a.dk_sh + (int64_t)key * a.dk_st;
    if (a.dv_accumulate) {
        Run4<DT> prev[MB][4];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int g = 0; g < 4; ++g) prev[mb][g] = Run4<DT>::load(dvr + 32 * mb + 8 * g + 4 * hi);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float x[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = dvt[mb][4 * g + e] + prev[mb][g].get(e);
                Run4<DT>::store(dvr + 32 * mb + 8 * g + 4 * hi, x);
            }
    } else {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float x[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = dvt[mb][4 * g + e];
                Run4<DT>::store(dvr + 32 * mb + 8 * g + 4 * hi, x);
            }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * rb + 8 * g + 4 * hi;
            if (d >= R) continue;
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = dkt[rb][4 * g + e] * a.sm_scale;
            Run4<DT>::store(dkr + d, x);
        }
}

template <int DT, int R, int D>
__global__ __launch_bounds__(NT, (dq_occupancy<DT, R, D>())) void attn_bwd_dq_kernel(AttnBwdK a) {
    using in_t = typename Stor<DT>::type;
    using LK = TileL<R>;
    using LV = TileL<D>;
    constexpr int KS = R / 16, DKS = D / 16;
    constexpr int RB = (R + 31) / 32;
    constexpr bool SPL = DT == HOFA_F32;
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][LK::ELEMS];
    __shared__ __attribute__((aligned(16))) uint16_t sKlo[2][SPL ? LK::ELEMS : 8];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][LV::ELEMS];

    const int nq = (a.T + BM - 1) / BM;
    int bh, qb;
    xcd_rank_remap(blockIdx.x, nq, a.B * a.H, &bh, &qb);
    qb = nq - 1 - qb;  // the last query blocks have the most work
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q0 = qb * BM, qw0 = q0 + 32 * w;
    const int qrow = qw0 + (lane & 31);

    const in_t *qp = (const in_t *)a.q + b * a.q_sb + h * a.q_sh;
    const in_t *kp = (const in_t *)a.k + b * a.k_sb + h * a.k_sh;
    const in_t *vp = (const in_t *)a.v + b * a.v_sb + h * a.v_sh;
    const in_t *op = (const in_t *)a.dO + b * a.o_sb + h * a.o_sh;
    TileStage<DT, R> stk;
    TileStage<DT, D> stv;
    TileDma<R> dmk;
    TileDma<D> dmv;
    if constexpr (!SPL) {
        dmk.init(kp, a.k_st, a.T, w, lane);
        dmv.init(vp, a.v_st, a.T, w, lane);
    }
    const int kend = min(a.T, q0 + BM);
    // the first tile's requests go out before the per-lane operands below, so
    // both arrive within one memory round trip
    if constexpr (SPL) {
        stk.fetch(kp, a.k_st, 0, a.T);
        stv.fetch(vp, a.v_st, 0, a.T);
    } else {
        dmk.fetch(sK[0], 0, w);
        dmv.fetch(sV[0], 0, w);
    }

    // B operands: c Q as a hi/lo pair (k = dims), dO (k = dv) of this lane's
    // query, and the shift k-step (-lse, -Dt) against ones
    u32x4 qh[KS], ql[KS], oop[DKS];
#pragma unroll
    for (int ks = 0; ks < DKS; ++ks)
        oop[ks] = qrow < a.T ? load_op8<DT>(op + (int64_t)qrow * a.o_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
    const float lq = qrow < a.T ? a.lse[(int64_t)bh * a.T + qrow] : 0.f;
    const float dq_t = qrow < a.T ? a.dt[(int64_t)bh * a.T + qrow] : 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        load_scaled_op8<DT>(qp + (int64_t)qrow * a.q_st + 16 * ks + 8 * hi, a.c, qrow < a.T, qh[ks], ql[ks]);
    const u32x4 xb = {hi ? 0u : split_pair<DT>(-lq), 0u, 0u, 0u};
    const u32x4 yb = {hi ? 0u : split_pair<DT>(-dq_t), 0u, 0u, 0u};
    const u32x4 ones = {hi ? 0u : kOnes2<DT>, 0u, 0u, 0u};

    f32x16 dqt[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int v = 0; v < 16; ++v) dqt[rb][v] = 0.f;

    if constexpr (SPL) {
        stk.put(sK[0], sKlo[0]);
        stv.put(sV[0], nullptr);
    } else {
        wait_vmem();
    }
    __syncthreads();
    auto tile = [&](int buf, int k0) {
        const bool more = k0 + BN < kend;
        if (more) {
            if constexpr (SPL) {
                stk.fetch(kp, a.k_st, k0 + BN, a.T);
                stv.fetch(vp, a.v_st, k0 + BN, a.T);
            } else {
                dmk.fetch(sK[buf ^ 1], k0 + BN, w);
                dmv.fetch(sV[buf ^ 1], k0 + BN, w);
            }
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int kk0 = k0 + 32 * kb;
            if (kk0 > qw0 + 31) continue;  // every key of the block follows this wave's queries
            const int rk = 32 * kb + (lane & 31);
            // this block's key rows: every row operand read is issued before the products
            u32x4 ka[KS], kla[SPL ? KS : 1], va[DKS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                ka[ks] = *(const u32x4 *)&sK[buf][LK::off(rk, 16 * ks + 8 * hi)];
                if constexpr (SPL) kla[ks] = *(const u32x4 *)&sKlo[buf][LK::off(rk, 16 * ks + 8 * hi)];
            }
#pragma unroll
            for (int ks = 0; ks < DKS; ++ks) va[ks] = *(const u32x4 *)&sV[buf][LV::off(rk, 16 * ks + 8 * hi)];
            // S'^T = c K Q^T - lse and dP'^T = V dO^T - Dt in C[key, query]
            f32x16 s = {}, dp = {};
            sched_reads_then_mfma<KS * (SPL ? 3 : 2) + 1, DKS + 1>();
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                s = mfma32<DT>(ka[ks], qh[ks], s);
                s = mfma32<DT>(ka[ks], ql[ks], s);
                if constexpr (SPL) s = mfma32<DT>(kla[ks], qh[ks], s);
            }
            s = mfma32<DT>(ones, xb, s);
#pragma unroll
            for (int ks = 0; ks < DKS; ++ks) dp = mfma32<DT>(va[ks], oop[ks], dp);
            dp = mfma32<DT>(ones, yb, dp);
            // blocks on the diagonal or past T: logits of keys past min(query, T-1) -> -inf
            if (kk0 + 31 > qw0 || kk0 + 31 >= a.T) {
                const int lim = min(qrow, a.T - 1) - kk0 - 4 * hi;  // key offset visible iff <= lim
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    if (8 * (v / 4) + (v % 4) > lim) s[v] = -INFINITY;
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) dp[v] *= fast_exp2(s[v]);
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const u32x4 db = pack8<DT>(dp, 8 * k2);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
                    dqt[rb] = mfma32<DT>(tr_operand<R>(sK[buf], 32 * kb + 16 * k2, 32 * rb, lane), db, dqt[rb]);
            }
        }
        if (more) {
            if constexpr (SPL) {
                stk.put(sK[buf ^ 1], sKlo[buf ^ 1]);
                stv.put(sV[buf ^ 1], nullptr);
            } else {
                wait_vmem();
            }
        }
        __syncthreads();
    };
    for (int k0 = 0, buf = 0; k0 < kend; k0 += BN, buf ^= 1) tile(buf, k0);
    if (qrow >= a.T) return;
    in_t *dqr = (in_t *)a.dq + b * a.dq_sb + h * a.dq_sh + (int64_t)qrow * a.dq_st;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * rb + 8 * g + 4 * hi;
            if (d >= R) continue;
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = dqt[rb][4 * g + e] * a.sm_scale;
            Run4<DT>::store(dqr + d, x);
        }
}

template <int DT, int R, int D>
void launch(const AttnBwdK &k, hipStream_t s) {
    const int nbh = k.B * k.H;
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<DT, R, D>), dim3(((k.T + BKB - 1) / BKB) * nbh), dim3(NT), 0, s, k);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<DT, R, D>), dim3(((k.T + BM - 1) / BM) * nbh), dim3(NT), 0, s, k);
}

template <int DT>
int dispatch(const AttnBwdK &k, int R, int D, hipStream_t s) {
    if (D == 64 && R == 16) launch<DT, 16, 64>(k, s);
    else if (D == 64 && R == 32) launch<DT, 32, 64>(k, s);
    else if (D == 64 && R == 64) launch<DT, 64, 64>(k, s);
    else if (D == 128 && R == 16) launch<DT, 16, 128>(k, s);
    else if (D == 128 && R == 32) launch<DT, 32, 128>(k, s);
    else if (D == 128 && R == 64) launch<DT, 64, 128>(k, s);
    else return HOFA_EUNSUPPORTED;
    return HOFA_OK;
}

int elem_bytes(int dt) { return dt == HOFA_F32 ? 4 : 2; }

bool rows_ok(const hofa_view_t &v, int es) {
    return v.stride[3] == 1 && ((uintptr_t)v.data % 16) == 0 && (v.stride[0] * es) % 16 == 0 &&
           (v.stride[1] * es) % 16 == 0 && (v.stride[2] * es) % 16 == 0;
}

}  // namespace
}  // namespace hofa

using namespace hofa;

extern "C" int hofa_attn_bwd(const hofa_attn_bwd_args_t *a, void *stream) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_attn_bwd: args is NULL");
    HOFA_REQUIRE(a->B > 0 && a->H > 0 && a->T > 0, HOFA_EINVAL, "hofa_attn_bwd: B=%d H=%d T=%d must be positive", a->B,
                 a->H, a->T);
    HOFA_REQUIRE(a->D == 64 || a->D == 128, HOFA_EUNSUPPORTED, "hofa_attn_bwd: head dim D=%d not in {64,128}", a->D);
    HOFA_REQUIRE((a->R == 16 || a->R == 32 || a->R == 64) && a->R <= a->D, HOFA_EUNSUPPORTED,
                 "hofa_attn_bwd: R=%d not in {16,32,64} or > D", a->R);
    const int dt = a->q.dtype;
    HOFA_REQUIRE(dt == HOFA_F32 || dt == HOFA_BF16 || dt == HOFA_F16, HOFA_EINVAL, "hofa_attn_bwd: bad dtype %d", dt);
    HOFA_REQUIRE(a->k.dtype == dt && a->v.dtype == dt && a->dout.dtype == dt && a->dq.dtype == dt &&
                     a->dk.dtype == dt && a->dv.dtype == dt,
                 HOFA_EINVAL, "hofa_attn_bwd: all tensors must share one dtype");
    HOFA_REQUIRE(a->q.data && a->k.data && a->v.data && a->dout.data && a->lse && a->delta && a->dq.data &&
                     a->dk.data && a->dv.data,
                 HOFA_EINVAL, "hofa_attn_bwd: NULL pointer");
    const int es = elem_bytes(dt);
    for (const hofa_view_t *v : {&a->q, &a->k, &a->v, &a->dout, &a->dq, &a->dk, &a->dv})
        HOFA_REQUIRE(rows_ok(*v, es), HOFA_EINVAL, "hofa_attn_bwd: tensors need unit last stride and 16-byte aligned rows");
    for (const hofa_view_t *v : {&a->q, &a->k, &a->v, &a->dout})
        HOFA_REQUIRE((int64_t)(a->T + 2 * BKB) * v->stride[2] * es < (1ll << 31), HOFA_EUNSUPPORTED,
                     "hofa_attn_bwd: one head's rows must span less than 2 GiB");
    AttnBwdK k{};
    k.q = a->q.data; k.k = a->k.data; k.v = a->v.data; k.dO = a->dout.data;
    k.lse = a->lse; k.dt = a->delta;
    k.dq = (void *)a->dq.data; k.dk = (void *)a->dk.data; k.dv = (void *)a->dv.data;
    k.q_sb = a->q.stride[0]; k.q_sh = a->q.stride[1]; k.q_st = a->q.stride[2];
    k.k_sb = a->k.stride[0]; k.k_sh = a->k.stride[1]; k.k_st = a->k.stride[2];
    k.v_sb = a->v.stride[0]; k.v_sh = a->v.stride[1]; k.v_st = a->v.stride[2];
    k.o_sb = a->dout.stride[0]; k.o_sh = a->dout.stride[1]; k.o_st = a->dout.stride[2];
    k.dq_sb = a->dq.stride[0]; k.dq_sh = a->dq.stride[1]; k.dq_st = a->dq.stride[2];
    k.dk_sb = a->dk.stride[0]; k.dk_sh = a->dk.stride[1]; k.dk_st = a->dk.stride[2];
    k.dv_sb = a->dv.stride[0]; k.dv_sh = a->dv.stride[1]; k.dv_st = a->dv.stride[2];
    k.B = a->B; k.H = a->H; k.T = a->T;
    k.dv_accumulate = a->dv_accumulate;
    k.c = a->sm_scale * kLog2e;
    k.sm_scale = a->sm_scale;
    hipStream_t s = (hipStream_t)stream;
    int rc;
    switch (dt) {
        case HOFA_F32: rc = dispatch<HOFA_F32>(k, a->R, a->D, s); break;
        case HOFA_BF16: rc = dispatch<HOFA_BF16>(k, a->R, a->D, s); break;
        default: rc = dispatch<HOFA_F16>(k, a->R, a->D, s); break;
    }
    if (rc) {
        set_error("hofa_attn_bwd: no kernel for this (R, D)");
        return rc;
    }
    return check_launch("hofa_attn_bwd");
}

// Outlier-pathway backward for gfx950: gradients of causal softmax attention
// with QK width R and value width D.
//
// No reference counterpart in the repository's own code: the reference
// trains through autograd of torch SDPA (src/HybridOutlierFactorizedAttentionTrain.py:258-259).
//
// With P = exp2(S * c - lse2) (c = sm_scale * log2(e)), dP = dO V^T,
// dS = P (.) (dP - Dt), Dt = rowsum(dO (.) O):
//   dV = P^T dO,  dK = sm_scale dS^T Q,  dQ = sm_scale dS K.
// Two kernels, no atomics:
//   attn_bwd_dkdv_kernel  block = 128 keys (4 waves x 32, lane = key), loop over
//                         the query tiles at or after the block; S, dP in the
//                         C[query, key] layout, so P and dS feed the dV^T and
//                         dK^T products straight from registers (A = dO^T, Q^T
//                         from LDS).
//   attn_bwd_dq_kernel    block = 128 queries (4 waves x 32, lane = query), loop
//                         over the key tiles up to the diagonal; S^T, dP^T in the
//                         C[key, query] layout, dQ^T = K^T dS^T.
// Matrix operands are 16-bit (bf16 for bf16/f32 inputs, f16 for f16) with f32
// accumulation, as in flash-attention backward passes; f32 inputs form the
// logits from hi/lo operand pairs so the recomputed probabilities agree with
// the forward's log-sum-exp.
#include "hofa_mfma.h"

namespace hofa {
namespace {

constexpr int NT = 256;
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

// Rows [t0, t0+64) of a [T, W] operand matrix, staged global -> registers
// (fetch, issued a tile ahead) -> LDS (put): row-major ([64][W + pad]) and/or
// transposed ([W][64 + pad]) 16-bit operands, rows past T zero; f32 inputs
// also keep their bf16 rounding remainders (row-major).  256 threads, each
// owning (2 rows x 8 columns) pieces.
template <int DT, int W>
struct RowStage {
    using in_t = typename Stor<DT>::type;
    static constexpr int NPIECE = 32 * (W / 8);
    static constexpr int NP = (NPIECE + NT - 1) / NT;
    static constexpr bool LO = DT == HOFA_F32;
    u32x4 x0[NP], x1[NP], l0[LO ? NP : 1], l1[LO ? NP : 1];

    __device__ void fetch(const in_t *base, int64_t st, int t0, int T) {
        const __amdgpu_buffer_rsrc_t r = rows_rsrc(base, (uint32_t)(T * st * sizeof(in_t)));
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int pi = min((int)threadIdx.x + NT * i, NPIECE - 1);  // extra threads repeat the last piece
            const int rp = pi / (W / 8), cc = pi % (W / 8);
            const uint32_t off = (uint32_t)(((t0 + 2 * rp) * st + 8 * cc) * sizeof(in_t));
            const uint32_t off1 = off + (uint32_t)(st * sizeof(in_t));
            if constexpr (LO) {
                x0[i] = bload_op8<DT>(r, off, &l0[i]);
                x1[i] = bload_op8<DT>(r, off1, &l1[i]);
            } else {
                x0[i] = bload16(r, off);
                x1[i] = bload16(r, off1);
            }
        }
    }
    template <int PR, int PT, bool ROW, bool TR>
    __device__ void put(uint16_t *row, uint16_t *tr, uint16_t *lo) const {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int pi = threadIdx.x + NT * i;
            if (pi >= NPIECE) continue;
            const int rp = pi / (W / 8), cc = pi % (W / 8);
            const int r0 = 2 * rp;
            if constexpr (ROW) {
                *(u32x4 *)&row[r0 * PR + 8 * cc] = x0[i];
                *(u32x4 *)&row[(r0 + 1) * PR + 8 * cc] = x1[i];
            }
            if constexpr (LO && ROW) {
                *(u32x4 *)&lo[r0 * PR + 8 * cc] = l0[i];
                *(u32x4 *)&lo[(r0 + 1) * PR + 8 * cc] = l1[i];
            }
            if constexpr (TR) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    *(uint32_t *)&tr[(8 * cc + 2 * e) * PT + r0] = __builtin_amdgcn_perm(x1[i][e], x0[i][e], 0x05040100u);
                    *(uint32_t *)&tr[(8 * cc + 2 * e + 1) * PT + r0] = __builtin_amdgcn_perm(x1[i][e], x0[i][e], 0x07060302u);
                }
            }
        }
    }
};

// A operand of a k-step of 16 along the permuted index of a C-layout tile:
// lane reads entries [16ks + 4hi .. +3] and [16ks + 8 + 4hi .. +3] of its row.
__device__ __forceinline__ u32x4 perm_a(const uint16_t *row, int ks, int hi) {
    const uint16_t *p = row + 16 * ks + 4 * hi;
    const uint2 lo = *(const uint2 *)p, h8 = *(const uint2 *)(p + 8);
    return u32x4{lo.x, lo.y, h8.x, h8.y};
}

template <int DT, int R, int D>
// Three waves per SIMD for the 16-bit d_h=64 kernels (LDS allows three blocks per CU).
__global__ __launch_bounds__(NT, (DT != HOFA_F32 && D == 64 && R <= 32) ? 3 : 1) void attn_bwd_dkdv_kernel(AttnBwdK a) {
    using in_t = typename Stor<DT>::type;
    constexpr int KS = R / 16, DKS = D / 16, MB = D / 32;
    constexpr int RB = (R + 31) / 32;  // 32-row blocks of dK^T
    constexpr int PQ = R + 8, PO = D + 8, PT = BQ + 4;
    constexpr bool SPL = DT == HOFA_F32;
    __shared__ __attribute__((aligned(16))) uint16_t sQ[2][BQ * PQ];
    __shared__ __attribute__((aligned(16))) uint16_t sQlo[2][SPL ? BQ * PQ : 8];
    __shared__ __attribute__((aligned(16))) uint16_t sQt[2][RB * 32 * PT];
    __shared__ __attribute__((aligned(16))) uint16_t sO[2][BQ * PO];
    __shared__ __attribute__((aligned(16))) uint16_t sOt[2][D * PT];
    __shared__ __attribute__((aligned(16))) float sL[2][BQ];
    __shared__ __attribute__((aligned(16))) float sD[2][BQ];

    const int nkb = (a.T + BKB - 1) / BKB;
    int bh, kblk;
    xcd_remap(blockIdx.x, nkb, a.B * a.H, &bh, &kblk);
    kblk = nkb - 1 - kblk;  // xcd_remap walks row blocks last-first; key blocks near 0 have the most work
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

    // B operands: K (k = dims) and V (k = dv) of this lane's key
    u32x4 kop[KS], klo[KS], vop[DKS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        kop[ks] = key < a.T ? load_op8<DT>(kp + (int64_t)key * a.k_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
        if constexpr (SPL)
            klo[ks] = key < a.T ? load_lo8_f32((const float *)kp + (int64_t)key * a.k_st + 16 * ks + 8 * hi)
                                : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int ks = 0; ks < DKS; ++ks)
        vop[ks] = key < a.T ? load_op8<DT>(vp + (int64_t)key * a.v_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
    // rows R..32*RB-1 of Q^T stay zero
    for (int i = tid; i < 2 * RB * 32 * PT; i += NT) (&sQt[0][0])[i] = 0;

    f32x16 dvt[MB], dkt[RB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) dvt[mb][v] = 0.f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int v = 0; v < 16; ++v) dkt[rb][v] = 0.f;

    RowStage<DT, R> stq;
    RowStage<DT, D> sto;
    float ls = 0.f, ds = 0.f;
    auto fetch = [&](int q0) {
        stq.fetch(qp, a.q_st, q0, a.T);
        sto.fetch(op, a.o_st, q0, a.T);
        if (tid < BQ) {
            ls = q0 + tid < a.T ? lse[q0 + tid] : 0.f;
            ds = q0 + tid < a.T ? dtp[q0 + tid] : 0.f;
        }
    };
    auto put = [&](int buf) {
        stq.template put<PQ, PT, true, true>(sQ[buf], sQt[buf], sQlo[buf]);
        sto.template put<PO, PT, true, true>(sO[buf], sOt[buf], nullptr);
        if (tid < BQ) {
            sL[buf][tid] = ls;
            sD[buf][tid] = ds;
        }
    };
    fetch(k0);
    __syncthreads();  // pad rows of Q^T cleared
    put(0);
    __syncthreads();
    int buf = 0;
    for (int q0 = k0; q0 < a.T; q0 += BQ, buf ^= 1) {
        const bool more = q0 + BQ < a.T;
        if (more) fetch(q0 + BQ);
        if (q0 + BQ - 1 >= kw0) {  // some query of the tile sees this wave's keys
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                f32x16 s = {}, dp = {};
                const uint16_t *qrow = &sQ[buf][(32 * qb + (lane & 31)) * PQ];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const u32x4 qa = *(const u32x4 *)(qrow + 16 * ks + 8 * hi);
                    s = mfma32<DT>(qa, kop[ks], s);
                    if constexpr (SPL) {
                        s = mfma32<DT>(qa, klo[ks], s);
                        s = mfma32<DT>(*(const u32x4 *)(&sQlo[buf][(32 * qb + (lane & 31)) * PQ] + 16 * ks + 8 * hi),
                                       kop[ks], s);
                    }
                }
                const uint16_t *orow = &sO[buf][(32 * qb + (lane & 31)) * PO];
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) dp = mfma32<DT>(*(const u32x4 *)(orow + 16 * ks + 8 * hi), vop[ks], dp);
                // P and dS in place (C[query, key]: lane = key, v -> query)
                const bool edge = q0 + 32 * qb < kw0 + 31 || q0 + 32 * qb + 31 >= a.T || kw0 + 31 >= a.T;
                // query offsets 8g + e of this lane (g = v/4, e = v%4) are visible iff vlo <= 8g + e <= vhi
                const int vlo = key - q0 - 32 * qb - 4 * hi;
                const int vhi = key < a.T ? a.T - 1 - q0 - 32 * qb - 4 * hi : -1;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 lq = *(const f32x4 *)&sL[buf][32 * qb + 8 * g + 4 * hi];
                    const f32x4 dq = *(const f32x4 *)&sD[buf][32 * qb + 8 * g + 4 * hi];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int v = 4 * g + e;
                        float p = fast_exp2(fmaf(s[v], a.c, -lq[e]));
                        if (edge) p = (8 * g + e >= vlo && 8 * g + e <= vhi) ? p : 0.f;
                        s[v] = p;
                        dp[v] = p * (dp[v] - dq[e]);
                    }
                }
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    const int ks4 = 2 * qb + k2;
                    const u32x4 pb = pack8<DT>(s, 8 * k2);
                    const u32x4 db = pack8<DT>(dp, 8 * k2);
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
                        dvt[mb] = mfma32<DT>(perm_a(&sOt[buf][(32 * mb + (lane & 31)) * PT], ks4, hi), pb, dvt[mb]);
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
                        dkt[rb] = mfma32<DT>(perm_a(&sQt[buf][(32 * rb + (lane & 31)) * PT], ks4, hi), db, dkt[rb]);
                }
            }
        }
        if (more) put(buf ^ 1);
        __syncthreads();
    }
    if (key >= a.T) return;
    // dV^T / dK^T: lane = key, rows 8(v/4) + 4hi + v%4 of each 32-row block
    in_t *dvr = (in_t *)a.dv + b * a.dv_sb + h * a.dv_sh + (int64_t)key * a.dv_st;
    in_t *dkr = (in_t *)a.dk + b * a.dk_sb + h * a.dk_sh + (int64_t)key * a.dk_st;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int d = 32 * mb + 8 * (v / 4) + 4 * hi + (v % 4);
            float x = dvt[mb][v];
            if (a.dv_accumulate) x += to_f32<DT>(dvr[d]);
            dvr[d] = from_f32<DT>(x);
        }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int d = 32 * rb + 8 * (v / 4) + 4 * hi + (v % 4);
            if (d < R) dkr[d] = from_f32<DT>(dkt[rb][v] * a.sm_scale);
        }
}

template <int DT, int R, int D>
__global__ __launch_bounds__(NT, (DT != HOFA_F32 && D == 64 && R <= 32) ? 4 : 1) void attn_bwd_dq_kernel(AttnBwdK a) {
    using in_t = typename Stor<DT>::type;
    constexpr int KS = R / 16, DKS = D / 16;
    constexpr int RB = (R + 31) / 32;
    constexpr int PK = R + 8, PV = D + 8, PT = BN + 4;
    constexpr bool SPL = DT == HOFA_F32;
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * PK];
    __shared__ __attribute__((aligned(16))) uint16_t sKlo[2][SPL ? BN * PK : 8];
    __shared__ __attribute__((aligned(16))) uint16_t sKt[2][RB * 32 * PT];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][BN * PV];

    const int nq = (a.T + BM - 1) / BM;
    int bh, qb;
    xcd_remap(blockIdx.x, nq, a.B * a.H, &bh, &qb);
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q0 = qb * BM, qw0 = q0 + 32 * w;
    const int qrow = qw0 + (lane & 31);

    const in_t *qp = (const in_t *)a.q + b * a.q_sb + h * a.q_sh;
    const in_t *kp = (const in_t *)a.k + b * a.k_sb + h * a.k_sh;
    const in_t *vp = (const in_t *)a.v + b * a.v_sb + h * a.v_sh;
    const in_t *op = (const in_t *)a.dO + b * a.o_sb + h * a.o_sh;
    u32x4 qop[KS], qlo[KS], oop[DKS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qop[ks] = qrow < a.T ? load_op8<DT>(qp + (int64_t)qrow * a.q_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
        if constexpr (SPL)
            qlo[ks] = qrow < a.T ? load_lo8_f32((const float *)qp + (int64_t)qrow * a.q_st + 16 * ks + 8 * hi)
                                 : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int ks = 0; ks < DKS; ++ks)
        oop[ks] = qrow < a.T ? load_op8<DT>(op + (int64_t)qrow * a.o_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
    const float lq = qrow < a.T ? a.lse[(int64_t)bh * a.T + qrow] : 0.f;
    const float dq_t = qrow < a.T ? a.dt[(int64_t)bh * a.T + qrow] : 0.f;
    for (int i = tid; i < 2 * RB * 32 * PT; i += NT) (&sKt[0][0])[i] = 0;

    f32x16 dqt[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int v = 0; v < 16; ++v) dqt[rb][v] = 0.f;

    RowStage<DT, R> stk;
    RowStage<DT, D> stv;
    const int kend = min(a.T, q0 + BM);
    stk.fetch(kp, a.k_st, 0, a.T);
    stv.fetch(vp, a.v_st, 0, a.T);
    __syncthreads();  // pad rows of K^T cleared
    stk.template put<PK, PT, true, true>(sK[0], sKt[0], sKlo[0]);
    stv.template put<PV, PT, true, false>(sV[0], nullptr, nullptr);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < kend; k0 += BN, buf ^= 1) {
        const bool more = k0 + BN < kend;
        if (more) {
            stk.fetch(kp, a.k_st, k0 + BN, a.T);
            stv.fetch(vp, a.v_st, k0 + BN, a.T);
        }
        if (k0 <= qw0 + 31) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                f32x16 s = {}, dp = {};
                const uint16_t *krow = &sK[buf][(32 * kb + (lane & 31)) * PK];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const u32x4 ka = *(const u32x4 *)(krow + 16 * ks + 8 * hi);
                    s = mfma32<DT>(ka, qop[ks], s);
                    if constexpr (SPL) {
                        s = mfma32<DT>(ka, qlo[ks], s);
                        s = mfma32<DT>(*(const u32x4 *)(&sKlo[buf][(32 * kb + (lane & 31)) * PK] + 16 * ks + 8 * hi),
                                       qop[ks], s);
                    }
                }
                const uint16_t *vrow = &sV[buf][(32 * kb + (lane & 31)) * PV];
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) dp = mfma32<DT>(*(const u32x4 *)(vrow + 16 * ks + 8 * hi), oop[ks], dp);
                const bool edge = k0 + 32 * kb + 31 > qw0 || k0 + 32 * kb + 31 >= a.T;
                const int lim = min(qrow, a.T - 1) - k0 - 32 * kb - 4 * hi;  // key offset visible iff <= lim
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float p = fast_exp2(fmaf(s[v], a.c, -lq));
                    if (edge) p = 8 * (v / 4) + (v % 4) <= lim ? p : 0.f;
                    dp[v] = p * (dp[v] - dq_t);
                }
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    const u32x4 db = pack8<DT>(dp, 8 * k2);
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
                        dqt[rb] = mfma32<DT>(perm_a(&sKt[buf][(32 * rb + (lane & 31)) * PT], 2 * kb + k2, hi), db, dqt[rb]);
                }
            }
        }
        if (more) {
            stk.template put<PK, PT, true, true>(sK[buf ^ 1], sKt[buf ^ 1], sKlo[buf ^ 1]);
            stv.template put<PV, PT, true, false>(sV[buf ^ 1], nullptr, nullptr);
        }
        __syncthreads();
    }
    if (qrow >= a.T) return;
    in_t *dqr = (in_t *)a.dq + b * a.dq_sb + h * a.dq_sh + (int64_t)qrow * a.dq_st;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int d = 32 * rb + 8 * (v / 4) + 4 * hi + (v % 4);
            if (d < R) dqr[d] = from_f32<DT>(dqt[rb][v] * a.sm_scale);
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

// Outlier-pathway prefill for gfx950: causal flash attention with QK width
// R (the outlier channels) and value width D, mixed into the output.
//
// Replaces exact_attention_triton / _fwd_kernel (src/exact_attention.py:46-188).
//
// Block = 4 waves x 32 query rows (BM = 128), keys in tiles of BN = 64,
// consumed as two 32-key halves.  Per half and wave:
//   S^T[key, query] = K_half Q^T            v_mfma_f32_32x32x16 (A = K from LDS, B = Q in registers;
//                                           f32 inputs add the hi*lo and lo*hi bf16 products)
//   P = exp2(c S - m)                       c = sm_scale log2 e; each lane owns one query row
//                                           (its 16 scores of the half sit in its registers and
//                                           in lane l^32), m = the row's reference max
//   O^T[dv, query] += V_half^T P^T          A = V^T read from the row-major V tile with the
//                                           transposing LDS load, B = P straight from the score
//                                           registers (keys in the order the load delivers them)
//   l[query] += sum P                       v_mfma_f32_16x16x32 of a 0/1 selector with the same
//                                           packed P operand: the row sums of the rounded P that
//                                           enters O, off the VALU (f32 inputs: an exact f32 sum
//                                           of the unrounded P)
// The next half's QK^T does not depend on this half's exponentials, so the
// matrix core and the VALU can overlap.  The reference max m is set by the
// first half and moves only when a later logit exceeds it by more than kTau
// (log2 units; P stays below 2^kTau), which rescales O and l.  A tile needs no
// row max at all when the Cauchy-Schwarz bound c |q| |k| (the key norms are
// taken while the tile is staged) is within m + kTau for every key of the tile
// and every row of the wave.
// K and V tiles are double-buffered in LDS, both row-major; the next tile's
// range-checked buffer loads are in flight while the current tile is consumed.
// K goes through registers (its squared row norms, v_dot2 of the packed
// operand with itself, are taken on the way); 16-bit V is written to LDS by
// the loads themselves (LDS DMA) in the swizzled 16-byte-granule layout whose
// row reads and transposing reads are free of bank conflicts, f32 V is
// rounded to bf16 in registers first.
#include <type_traits>

#include "hofa_tile.h"

namespace hofa {
namespace {

constexpr int BM = 128, BN = 64, NT = 256;

struct AttnFwdK {
    const void *q, *k, *v, *mix;
    void *y, *o;
    float *lse;
    const float *acc;  // optional f32 partial: y = acc + mix * O
    int64_t a_sb, a_sh, a_st;
    int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st;
    int64_t y_sb, y_sh, y_st, o_sb, o_sh, o_st;
    int64_t m_sb, m_sh, m_st;
    int mix_dt;
    int B, H, T;
    int accumulate;
    float c;  // sm_scale * log2(e)
};

// x(l) + x(l ^ 32) and max(x(l), x(l ^ 32)) for every lane: one
// v_permlane32_swap of x with itself puts both halves side by side (either
// way round, so the sum / max is the same).
__device__ __forceinline__ float xor32_sum(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xor32_max(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Sum over each group of N consecutive lanes (N = 1, 2, 4 within quads via
// DPP; 8 adds one swizzle), without a round trip through LDS for N <= 4.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (N >= 2) x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
    if constexpr (N >= 4) x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
    if constexpr (N >= 8) x += __shfl_xor(x, 4);
    return x;
}

// acc + |x|^2 for a dword of two 16-bit key elements (v_dot2 of x with itself).
template <int DT>
__device__ __forceinline__ float dot2_self(uint32_t x, float acc) {
    if constexpr (kF16Ops<DT>)
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), __builtin_bit_cast(f16x2, x), acc, false);
    else
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), __builtin_bit_cast(bf16x2, x), acc,
                                               false);
}

template <int DT, int R, int D>
__global__ __launch_bounds__(NT, (D == 64 && R <= 32) ? 4 : 2) void attn_fwd_kernel(AttnFwdK a) {
    using in_t = typename Stor<DT>::type;
    constexpr int KS = R / 16;       // MFMA k-steps of S^T
    constexpr int MB = D / 32;       // 32-row blocks of O^T
    constexpr int KP = R + 8;        // K tile pitch in LDS (elements)
    constexpr int KCH = BN * R / 8;  // 16-byte K chunks per tile
    constexpr int NKC = (KCH + NT - 1) / NT;
    constexpr bool SPLIT = DT == HOFA_F32;      // logits from split-bf16 operands
    constexpr int KLO = SPLIT ? BN * KP : 0;    // offset of the K remainder tile
    constexpr float kTau = kF16Ops<DT> ? 15.f : 64.f;  // P <= 2^kTau (f16 operands: below 65504)
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * KP + KLO];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][tile::TileL<D>::ELEMS];  // V row-major, keys = rows
    __shared__ float sKn[2][BN];  // squared norm of every key row of each tile

    // One row block per block, dispatched longest first (row block nq - 1 has
    // the most causal work): the blocks that start last are the short ones,
    // and they fill the CUs that the long ones leave free.
    const int nq = (a.T + BM - 1) / BM;
    int bh, rank;
    xcd_rank_remap(blockIdx.x, nq, a.B * a.H, &bh, &rank);
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;  // which half of the wave
    const int qb = nq - 1 - rank;
    const int q0 = qb * BM;
    const int qw0 = q0 + 32 * w;  // first query row of this wave
    const int qrow = qw0 + (lane & 31);

    const in_t *qp = (const in_t *)a.q + b * a.q_sb + h * a.q_sh;
    const in_t *kp = (const in_t *)a.k + b * a.k_sb + h * a.k_sh;
    const in_t *vp = (const in_t *)a.v + b * a.v_sb + h * a.v_sh;

    // B operand Q (f32 inputs: hi/lo), loaded once the first tile's loads are issued
    u32x4 qop[KS], qlo[KS];

    const int kend = min(a.T, q0 + BM);
    const int ntiles = (kend + BN - 1) / BN;

    // ---- cooperative tile loader (global -> registers -> LDS): the next tile's
    // loads are in flight while the current tile is consumed
    u32x4 kreg[NKC], klo[NKC];
    // V: 16-bit inputs by LDS DMA straight into the tile image, f32 inputs
    // through registers (rounded to the bf16 operand)
    constexpr bool VDMA = DT != HOFA_F32;
    tile::TileDma<D> vdma;
    tile::TileStage<DT, D, false> vstage;
    if constexpr (VDMA) vdma.init(vp, a.v_st, a.T, w, lane);
    int vtr[MB][2];  // lane offsets of the transposing V^T operand reads
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 2; ++j) vtr[mb][j] = tile::tr_lane_off<D>(32 * mb, lane, j);
    constexpr int ES = sizeof(in_t);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kp, (uint32_t)(a.T * a.k_st * ES));
    auto gload = [&](int kt) {
        const int k0 = kt * BN;
#pragma unroll
        for (int i = 0; i < NKC; ++i) {
            const int ci = min(tid + NT * i, KCH - 1);  // threads past the tile reload its last chunk
            const int row = ci / (R / 8), part = ci % (R / 8);
            const uint32_t off = (uint32_t)(((k0 + row) * a.k_st + 8 * part) * ES);
            kreg[i] = bload_op8<DT>(rk, off, SPLIT ? &klo[i] : nullptr);
        }
        if constexpr (VDMA) vdma.fetch(sV[kt & 1], k0, w);
        else vstage.fetch(vp, a.v_st, k0, a.T);
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NKC; ++i) {
            const int ci = tid + NT * i;
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (SPLIT) {
                    const float x0 = op_to_f32<DT>(kreg[i][e] & 0xffffu) + op_to_f32<DT>(klo[i][e] & 0xffffu);
                    const float x1 = op_to_f32<DT>(kreg[i][e] >> 16) + op_to_f32<DT>(klo[i][e] >> 16);
                    ss = fmaf(x0, x0, fmaf(x1, x1, ss));
                } else {
                    ss = dot2_self<DT>(kreg[i][e], ss);
                }
            }
            ss = group_sum<R / 8>(ss);  // the row's chunks sit in R/8 consecutive lanes
            if (ci < KCH) {
                const int row = ci / (R / 8), part = ci % (R / 8);
                if (part == 0) sKn[buf][row] = ss;
                *(u32x4 *)&sK[buf][row * KP + 8 * part] = kreg[i];
                if constexpr (SPLIT) *(u32x4 *)&sK[buf][KLO + row * KP + 8 * part] = klo[i];
            }
        }
        if constexpr (!VDMA) vstage.put(sV[buf], nullptr);
        else tile::wait_vmem();  // this wave's share of the V tile has landed
    };

    float mref = -INFINITY;  // reference max of the scaled logits (base 2)
    f32x16 o[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[mb][v] = 0.f;
    float lsum = 0.f;  // f32 inputs: this lane's part of the row sum (the partner lane l^32 holds the rest)
    // 16-bit P: the row sums come from the matrix core, a 16x16x32 product of
    // a selector A (row 0: ones on k-groups 0 and 2, row 1: ones on groups 1
    // and 3) with the packed P operand, whose k-groups 0/2 hold queries
    // l % 16 and 1/3 queries 16 + l % 16: C[0][j] sums query j, C[1][j] query 16 + j
    f32x4 lacc = {0.f, 0.f, 0.f, 0.f};
    const uint32_t selw = ((lane & 15) == ((lane >> 4) & 1) && (lane & 15) < 2) ? tile::kOnes2<DT> : 0u;
    const u32x4 sel = {selw, selw, selw, selw};

    // One 32-key half (keys k0 .. k0+31, all at or before every query row of
    // the wave unless MASK).  EXACT forms the row max and moves the reference
    // (rescaling O and l) when a logit exceeds it by more than kTau; without
    // EXACT the caller has shown with the Cauchy-Schwarz bound that no logit
    // does, and the half runs without branches.
    auto half = [&](int buf, int kb, int k0, auto exact, auto mask) {
        f32x16 s = {};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 ka = *(const u32x4 *)&sK[buf][(32 * kb + (lane & 31)) * KP + 16 * ks + 8 * hi];
            s = mfma32<DT>(ka, qop[ks], s);
            if constexpr (SPLIT) {
                const u32x4 kl = *(const u32x4 *)&sK[buf][KLO + (32 * kb + (lane & 31)) * KP + 16 * ks + 8 * hi];
                s = mfma32<DT>(ka, qlo[ks], s);
                s = mfma32<DT>(kl, qop[ks], s);
            }
        }
        if constexpr (decltype(mask)::value) {  // causal mask (keys past T are past every valid row)
            const int lim = qrow - k0 - 4 * hi;  // visible iff row offset <= lim
#pragma unroll
            for (int v = 0; v < 16; ++v) s[v] = 8 * (v / 4) + (v % 4) <= lim ? s[v] : -INFINITY;
        }
        if constexpr (decltype(exact)::value) {
            float t4[4];  // the max as a tree (short dependency chains)
#pragma unroll
            for (int i = 0; i < 4; ++i) t4[i] = fmaxf(fmaxf(s[i], s[i + 4]), fmaxf(s[i + 8], s[i + 12]));
            float mx = fmaxf(fmaxf(t4[0], t4[1]), fmaxf(t4[2], t4[3]));
            mx = xor32_max(mx) * a.c;  // every row sees at least one key of the half
            if (__ballot(mx > mref + kTau)) {  // (re)set the reference: rescale O and l
                const float mn = mx > mref + kTau ? mx : mref;
                const float alpha = fast_exp2(mref - mn);  // 0 while O and l are still empty
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) o[mb] *= alpha;
                if constexpr (SPLIT) {
                    lsum *= alpha;
                } else {  // lacc[1] of lane j < 16 belongs to query 16 + j, whose alpha lane 16 + j holds
                    const float a16 = __shfl(alpha, (lane & 15) + 16);
                    lacc[0] *= alpha;
                    lacc[1] *= a16;
                }
                mref = mn;
            }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) s[v] = fast_exp2(fmaf(s[v], a.c, -mref));
        if constexpr (SPLIT) {
            float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int v = 0; v < 16; ++v) ps[v % 4] += s[v];
            lsum += (ps[0] + ps[1]) + (ps[2] + ps[3]);
        }
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            const int ks4 = 2 * kb + k2;
            const u32x4 pb = pack8<DT>(s, 8 * k2);
            if constexpr (!SPLIT) lacc = mfma16<DT>(sel, pb, lacc);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const uint16_t *vt = sV[buf] + 16 * ks4 * tile::TileL<D>::PITCH;  // V^T operand (tr_operand)
                const uint2 v0 = tile::lds_tr16(vt + vtr[mb][0]), v1 = tile::lds_tr16(vt + vtr[mb][1]);
                const u32x4 va = {v0.x, v0.y, v1.x, v1.y};
                o[mb] = mfma32<DT>(va, pb, o[mb]);
            }
        }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;

    // Tiles [0, nfull) lie at or before the first query row of the block, so
    // every key is visible to every row; the last one or two tiles hold the
    // diagonal.  Each loop iteration has one barrier, whichever loop a wave is
    // in, so the waves of the block stay in step through the tile staging.
    const int nfull = min(q0 / BN, ntiles);
    gload(0);
    // Q after the first tile's K and V requests, so all three share one memory
    // round trip; qn = c |q| with a relative 2^-10 margin
    float qss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qop[ks] = qrow < a.T ? load_op8<DT>(qp + (int64_t)qrow * a.q_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
        if constexpr (SPLIT)
            qlo[ks] = qrow < a.T ? load_lo8_f32((const float *)qp + (int64_t)qrow * a.q_st + 16 * ks + 8 * hi)
                                 : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float x0 = op_to_f32<DT>(qop[ks][e] & 0xffffu), x1 = op_to_f32<DT>(qop[ks][e] >> 16);
            if constexpr (SPLIT) {
                x0 += op_to_f32<DT>(qlo[ks][e] & 0xffffu);
                x1 += op_to_f32<DT>(qlo[ks][e] >> 16);
            }
            qss = fmaf(x0, x0, fmaf(x1, x1, qss));
        }
    }
    const float qn = __builtin_amdgcn_sqrtf(xor32_sum(qss)) * (a.c * (1.f + 1.f / 1024.f));
    lstore(0);
    __syncthreads();
    // The fast run needs no row max while every key k of the tile and every row
    // q of the wave satisfy c |q| |k| + 2^-6 <= m_q + kTau, i.e. while
    // |k|^2 <= theta2 = (min over rows of (m_q + kTau - 2^-6) / (c |q|))^2;
    // theta2 changes only when a reference moves (after an exact tile).
    float theta2 = -1.f;  // no reference yet: the first tile is exact
    auto update_theta = [&]() {
        float t = qn > 0.f ? (mref + kTau - 1.f / 64.f) / qn : INFINITY;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) t = fminf(t, __shfl_xor(t, off));
        theta2 = t >= 0.f ? t * t : -1.f;
    };
    int kt = 0;
    while (kt < nfull) {
        for (; kt < nfull; ++kt) {  // fast run
            if (__ballot(sKn[kt & 1][lane] > theta2)) break;  // lane = key row of the tile; wave-uniform
            const bool more = kt + 1 < ntiles;
            if (more) gload(kt + 1);
            half(kt & 1, 0, kt * BN, F_{}, F_{});
            half(kt & 1, 1, kt * BN + 32, F_{}, F_{});
            if (more) lstore((kt + 1) & 1);
            __syncthreads();
        }
        if (kt == nfull) break;
        // one tile with the exact row max (sets or moves the reference)
        const bool more = kt + 1 < ntiles;
        if (more) gload(kt + 1);
        half(kt & 1, 0, kt * BN, T_{}, F_{});
        half(kt & 1, 1, kt * BN + 32, T_{}, F_{});
        if (more) lstore((kt + 1) & 1);
        __syncthreads();
        update_theta();
        ++kt;
    }
    // the diagonal tiles: per half, fully visible (k0 < qw0), diagonal (k0 == qw0) or past the wave
    for (; kt < ntiles; ++kt) {
        const bool more = kt + 1 < ntiles;
        if (more) gload(kt + 1);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int k0 = kt * BN + 32 * kb;
            if (k0 < qw0) half(kt & 1, kb, k0, T_{}, F_{});
            else if (k0 == qw0) half(kt & 1, kb, k0, T_{}, T_{});
        }
        if (more) lstore((kt + 1) & 1);
        __syncthreads();
    }

    // ---- epilogue: y (+)= mix * O, optional O and lse
    float l;
    if constexpr (SPLIT) {
        l = xor32_sum(lsum);
    } else {
        const int src = lane & 15;
        const float l0 = __shfl(lacc[0], src), l1 = __shfl(lacc[1], src);
        l = (lane & 16) ? l1 : l0;
    }
    if (qrow >= a.T) return;
    const float inv = 1.f / l;
    const float mixv = a.mix ? load_any(a.mix, a.mix_dt, b * a.m_sb + h * a.m_sh + (int64_t)qrow * a.m_st) : 1.f;
    in_t *yr = (in_t *)a.y + b * a.y_sb + h * a.y_sh + (int64_t)qrow * a.y_st;
    in_t *orow = a.o ? (in_t *)a.o + b * a.o_sb + h * a.o_sh + (int64_t)qrow * a.o_st : nullptr;
    const float *arow = a.acc ? a.acc + b * a.a_sb + h * a.a_sh + (int64_t)qrow * a.a_st : nullptr;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int dv = 32 * mb + 8 * g + 4 * hi;
            float ov[4], yv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ov[e] = o[mb][4 * g + e] * inv;
                yv[e] = mixv * ov[e];
            }
            if (arow) {
                const f32x4 p = *(const f32x4 *)(arow + dv);
#pragma unroll
                for (int e = 0; e < 4; ++e) yv[e] += p[e];
            } else if (a.accumulate) {
                if constexpr (DT == HOFA_F32) {
                    const f32x4 p = *(const f32x4 *)(yr + dv);
#pragma unroll
                    for (int e = 0; e < 4; ++e) yv[e] += p[e];
                } else {
                    const uint2 p = *(const uint2 *)(yr + dv);
                    yv[0] += to_f32<DT>((uint16_t)(p.x & 0xffffu));
                    yv[1] += to_f32<DT>((uint16_t)(p.x >> 16));
                    yv[2] += to_f32<DT>((uint16_t)(p.y & 0xffffu));
                    yv[3] += to_f32<DT>((uint16_t)(p.y >> 16));
                }
            }
            if constexpr (DT == HOFA_F32) {
                *(f32x4 *)(yr + dv) = f32x4{yv[0], yv[1], yv[2], yv[3]};
                if (orow) *(f32x4 *)(orow + dv) = f32x4{ov[0], ov[1], ov[2], ov[3]};
            } else {
                *(uint2 *)(yr + dv) = uint2{pack2<DT>(yv[0], yv[1]), pack2<DT>(yv[2], yv[3])};
                if (orow) *(uint2 *)(orow + dv) = uint2{pack2<DT>(ov[0], ov[1]), pack2<DT>(ov[2], ov[3])};
            }
        }
    if (a.lse && hi == 0) a.lse[(int64_t)bh * a.T + qrow] = mref + __log2f(l);
}

template <int DT, int R, int D>
void launch(const AttnFwdK &k, hipStream_t s) {
    const int nq = (k.T + BM - 1) / BM;
    hipLaunchKernelGGL((attn_fwd_kernel<DT, R, D>), dim3(nq * k.B * k.H), dim3(NT), 0, s, k);
}

template <int DT>
int dispatch(const AttnFwdK &k, int R, int D, hipStream_t s) {
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

extern "C" int hofa_attn_fwd(const hofa_attn_fwd_args_t *a, void *stream) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_attn_fwd: args is NULL");
    HOFA_REQUIRE(a->B > 0 && a->H > 0 && a->T > 0, HOFA_EINVAL, "hofa_attn_fwd: B=%d H=%d T=%d must be positive", a->B,
                 a->H, a->T);
    HOFA_REQUIRE(a->D == 64 || a->D == 128, HOFA_EUNSUPPORTED, "hofa_attn_fwd: head dim D=%d not in {64,128}", a->D);
    HOFA_REQUIRE((a->R == 16 || a->R == 32 || a->R == 64) && a->R <= a->D, HOFA_EUNSUPPORTED,
                 "hofa_attn_fwd: R=%d not in {16,32,64} or > D", a->R);
    const int dt = a->q.dtype;
    HOFA_REQUIRE(dt == HOFA_F32 || dt == HOFA_BF16 || dt == HOFA_F16, HOFA_EINVAL, "hofa_attn_fwd: bad dtype %d", dt);
    HOFA_REQUIRE(a->k.dtype == dt && a->v.dtype == dt && a->y.dtype == dt && (!a->o.data || a->o.dtype == dt),
                 HOFA_EINVAL, "hofa_attn_fwd: q, k, v, y and o must share one dtype");
    HOFA_REQUIRE(a->q.data && a->k.data && a->v.data && a->y.data, HOFA_EINVAL, "hofa_attn_fwd: NULL tensor pointer");
    const int es = elem_bytes(dt);
    HOFA_REQUIRE(rows_ok(a->q, es) && rows_ok(a->k, es) && rows_ok(a->v, es) && rows_ok(a->y, es) &&
                     (!a->o.data || rows_ok(a->o, es)),
                 HOFA_EINVAL, "hofa_attn_fwd: q/k/v/y/o need unit last stride and 16-byte aligned rows");
    HOFA_REQUIRE(!a->mix.data || a->mix.dtype == HOFA_F32 || a->mix.dtype == HOFA_BF16 || a->mix.dtype == HOFA_F16,
                 HOFA_EINVAL, "hofa_attn_fwd: bad mix dtype");
    HOFA_REQUIRE(!a->acc.data || (a->acc.dtype == HOFA_F32 && rows_ok(a->acc, 4)), HOFA_EINVAL,
                 "hofa_attn_fwd: acc must be float32 with unit last stride and 16-byte aligned rows");
    HOFA_REQUIRE((int64_t)(a->T + 2 * BN) * a->k.stride[2] * es < (1ll << 31) &&
                     (int64_t)(a->T + 2 * BN) * a->v.stride[2] * es < (1ll << 31),
                 HOFA_EUNSUPPORTED, "hofa_attn_fwd: one head's K/V rows must span less than 2 GiB");
    AttnFwdK k{};
    k.q = a->q.data; k.k = a->k.data; k.v = a->v.data; k.mix = a->mix.data;
    k.y = (void *)a->y.data; k.o = (void *)a->o.data; k.lse = a->lse;
    k.acc = (const float *)a->acc.data;
    k.a_sb = a->acc.stride[0]; k.a_sh = a->acc.stride[1]; k.a_st = a->acc.stride[2];
    k.q_sb = a->q.stride[0]; k.q_sh = a->q.stride[1]; k.q_st = a->q.stride[2];
    k.k_sb = a->k.stride[0]; k.k_sh = a->k.stride[1]; k.k_st = a->k.stride[2];
    k.v_sb = a->v.stride[0]; k.v_sh = a->v.stride[1]; k.v_st = a->v.stride[2];
    k.y_sb = a->y.stride[0]; k.y_sh = a->y.stride[1]; k.y_st = a->y.stride[2];
    k.o_sb = a->o.stride[0]; k.o_sh = a->o.stride[1]; k.o_st = a->o.stride[2];
    k.m_sb = a->mix.stride[0]; k.m_sh = a->mix.stride[1]; k.m_st = a->mix.stride[2];
    k.mix_dt = a->mix.dtype;
    k.B = a->B; k.H = a->H; k.T = a->T;
    k.accumulate = a->accumulate;
    k.c = a->sm_scale * kLog2e;
    hipStream_t s = (hipStream_t)stream;
    int rc;
    switch (dt) {
        case HOFA_F32: rc = dispatch<HOFA_F32>(k, a->R, a->D, s); break;
        case HOFA_BF16: rc = dispatch<HOFA_BF16>(k, a->R, a->D, s); break;
        default: rc = dispatch<HOFA_F16>(k, a->R, a->D, s); break;
    }
    if (rc) {
        set_error("hofa_attn_fwd: no kernel for this (R, D)");
        return rc;
    }
    return check_launch("hofa_attn_fwd");
}

// Outlier-pathway prefill for gfx950: causal flash attention with QK width
// R (the outlier channels) and value width D, mixed into the output.
//
// Replaces exact_attention_triton / _fwd_kernel (src/exact_attention.py:46-188).
//
// Block = 4 waves x 32 query rows (BM = 128), keys in tiles of BN = 64.
// Per tile and wave:
//   S^T[key, query] = K_tile Q^T            v_mfma_f32_32x32x16 (A = K from LDS, B = Q in registers;
//                                           f32 inputs add the hi*lo and lo*hi bf16 products)
//   online softmax in the base-2 domain     each lane owns one query row: its 32 scores of a
//                                           tile sit in its registers and in lane l^32
//   O^T[dv, query] += V_tile^T P^T          A = V^T from LDS (stored transposed), B = P straight
//                                           from the score registers (keys permuted consistently)
//   l[query] += 1^T P^T                     the row sum on the matrix core (A = ones), over the
//                                           same rounded P that enters O (f32 inputs: an exact f32
//                                           sum of the unrounded P)
// so the row max and the rescale of O never leave a lane pair.  The rescale
// is lazy: the reference max moves only when a tile's max exceeds it by more
// than kTau (log2 units), so P stays below 2^kTau and O is rarely rescaled.
// K (row-major) and V^T tiles are double-buffered in LDS; the next tile's
// range-checked buffer loads are in flight while the current tile is consumed.
#include "hofa_mfma.h"

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

template <int DT, int R, int D>
__global__ __launch_bounds__(NT, (D == 64 && R <= 32) ? 4 : 2) void attn_fwd_kernel(AttnFwdK a) {
    using in_t = typename Stor<DT>::type;
    constexpr int KS = R / 16;       // MFMA k-steps of S^T
    constexpr int MB = D / 32;       // 32-row blocks of O^T
    constexpr int KP = R + 8;        // K tile pitch in LDS (elements)
    constexpr int VP = BN + 4;       // V^T tile pitch in LDS (elements)
    constexpr int KCH = BN * R / 8;  // 16-byte K chunks per tile
    constexpr int NKC = (KCH + NT - 1) / NT;
    constexpr int NVP = (BN / 2) * (D / 8) / NT;  // (2 keys x 8 dv) pieces of V per thread
    static_assert(NVP >= 1 && (BN / 2) * (D / 8) % NT == 0, "V tile split");
    constexpr bool SPLIT = DT == HOFA_F32;         // logits from split-bf16 operands
    constexpr int KLO = SPLIT ? BN * KP : 0;      // offset of the K remainder tile
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * KP + KLO];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][D * VP];

    const int nq = (a.T + BM - 1) / BM;
    int bh, qb;
    xcd_remap(blockIdx.x, nq, a.B * a.H, &bh, &qb);
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;  // which half of the wave
    const int q0 = qb * BM;
    const int qw0 = q0 + 32 * w;  // first query row of this wave
    const int qrow = qw0 + (lane & 31);

    const in_t *qp = (const in_t *)a.q + b * a.q_sb + h * a.q_sh;
    const in_t *kp = (const in_t *)a.k + b * a.k_sb + h * a.k_sh;
    const in_t *vp = (const in_t *)a.v + b * a.v_sb + h * a.v_sh;

    u32x4 qop[KS], qlo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qop[ks] = qrow < a.T ? load_op8<DT>(qp + (int64_t)qrow * a.q_st + 16 * ks + 8 * hi) : u32x4{0, 0, 0, 0};
        if constexpr (SPLIT)
            qlo[ks] = qrow < a.T ? load_lo8_f32((const float *)qp + (int64_t)qrow * a.q_st + 16 * ks + 8 * hi)
                                 : u32x4{0, 0, 0, 0};
    }

    const int kend = min(a.T, q0 + BM);
    const int ntiles = (kend + BN - 1) / BN;

    // ---- cooperative tile loader (global -> registers -> LDS): the next tile's
    // loads are in flight while the current tile is consumed
    u32x4 kreg[1][NKC], klo[1][NKC];
    u32x4 vreg[1][NVP][2];
    constexpr int ES = sizeof(in_t);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kp, (uint32_t)(a.T * a.k_st * ES));
    const __amdgpu_buffer_rsrc_t rv = rows_rsrc(vp, (uint32_t)(a.T * a.v_st * ES));
    auto gload = [&](int kt, int sl) {
        const int k0 = kt * BN;
#pragma unroll
        for (int i = 0; i < NKC; ++i) {
            const int ci = min(tid + NT * i, KCH - 1);  // threads past the tile reload its last chunk
            const int row = ci / (R / 8), part = ci % (R / 8);
            const uint32_t off = (uint32_t)(((k0 + row) * a.k_st + 8 * part) * ES);
            kreg[sl][i] = bload_op8<DT>(rk, off, SPLIT ? &klo[sl][i] : nullptr);
        }
#pragma unroll
        for (int i = 0; i < NVP; ++i) {
            const int pi = tid + NT * i;
            const int kpair = pi / (D / 8), cch = pi % (D / 8);
            const uint32_t off = (uint32_t)(((k0 + 2 * kpair) * a.v_st + 8 * cch) * ES);
            vreg[sl][i][0] = bload_op8<DT>(rv, off);
            vreg[sl][i][1] = bload_op8<DT>(rv, off + (uint32_t)(a.v_st * ES));
        }
    };
    auto lstore = [&](int buf, int sl) {
#pragma unroll
        for (int i = 0; i < NKC; ++i) {
            const int ci = tid + NT * i;
            if (ci < KCH) {
                const int row = ci / (R / 8), part = ci % (R / 8);
                *(u32x4 *)&sK[buf][row * KP + 8 * part] = kreg[sl][i];
                if constexpr (SPLIT) *(u32x4 *)&sK[buf][KLO + row * KP + 8 * part] = klo[sl][i];
            }
        }
#pragma unroll
        for (int i = 0; i < NVP; ++i) {
            const int pi = tid + NT * i;
            const int kpair = pi / (D / 8), cch = pi % (D / 8);
            // transpose a (2 keys x 8 dv) piece: dv row gets the key pair as one dword
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t x0 = vreg[sl][i][0][e], x1 = vreg[sl][i][1][e];
                *(uint32_t *)&sV[buf][(8 * cch + 2 * e) * VP + 2 * kpair] = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
                *(uint32_t *)&sV[buf][(8 * cch + 2 * e + 1) * VP + 2 * kpair] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
            }
        }
    };

    constexpr float kTau = 8.f;
    constexpr uint32_t kOne2 = kF16Ops<DT> ? 0x3C003C00u : 0x3F803F80u;  // two 16-bit 1.0
    const u32x4 ones = {kOne2, kOne2, kOne2, kOne2};
    float mref = -INFINITY;  // reference max of the scaled logits (base 2)
    f32x16 o[MB], lacc;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[mb][v] = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) lacc[v] = 0.f;

    float lsum = 0.f;  // f32 inputs: exact row sum of the unrounded probabilities
    auto tile = [&](int kt, int buf) {
        const int k0 = kt * BN;
        if (k0 > qw0 + 31) return;  // every key of this tile is after this wave's queries
        f32x16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            s[kb] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const u32x4 ka = *(const u32x4 *)&sK[buf][(32 * kb + (lane & 31)) * KP + 16 * ks + 8 * hi];
                s[kb] = mfma32<DT>(ka, qop[ks], s[kb]);
                if constexpr (SPLIT) {
                    const u32x4 kl = *(const u32x4 *)&sK[buf][KLO + (32 * kb + (lane & 31)) * KP + 16 * ks + 8 * hi];
                    s[kb] = mfma32<DT>(ka, qlo[ks], s[kb]);
                    s[kb] = mfma32<DT>(kl, qop[ks], s[kb]);
                }
            }
        }
        if (k0 + BN - 1 > qw0 || k0 + BN > a.T) {  // tile crosses the diagonal or the end
            const int lim = min(qrow, a.T - 1) - k0 - 4 * hi;  // visible iff row offset <= lim
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    s[kb][v] = 32 * kb + 8 * (v / 4) + (v % 4) <= lim ? s[kb][v] : -INFINITY;
        }
        float t8[8];  // max as a tree (short dependency chains)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            t8[i] = fmaxf(fmaxf(s[0][i], s[0][i + 8]), fmaxf(s[1][i], s[1][i + 8]));
#pragma unroll
        for (int i = 0; i < 4; ++i) t8[i] = fmaxf(t8[i], t8[i + 4]);
        float mx = fmaxf(fmaxf(t8[0], t8[1]), fmaxf(t8[2], t8[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 32)) * a.c;
        if (__ballot(mx > mref + kTau)) {  // some row's max moved far: rescale (wave-uniform branch)
            const float mn = fmaxf(mref, mx);
            const float alpha = fast_exp2(mref - mn);  // 0 on the first tile (mref = -inf)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) o[mb] *= alpha;
            if constexpr (SPLIT) lsum *= alpha;
            else lacc *= alpha;
            mref = mn;
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v) s[kb][v] = fast_exp2(fmaf(s[kb][v], a.c, -mref));
        if constexpr (SPLIT) {
            float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) ps[v % 4] += s[kb][v];
            lsum += (ps[0] + ps[1]) + (ps[2] + ps[3]);
        }
#pragma unroll
        for (int ks4 = 0; ks4 < 4; ++ks4) {
            const u32x4 pb = pack8<DT>(s[ks4 / 2], 8 * (ks4 % 2));
            if constexpr (!SPLIT) lacc = mfma32<DT>(ones, pb, lacc);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const uint16_t *vr = &sV[buf][(32 * mb + (lane & 31)) * VP + 16 * ks4 + 4 * hi];
                const uint2 lo = *(const uint2 *)vr, hi8 = *(const uint2 *)(vr + 8);
                const u32x4 va = {lo.x, lo.y, hi8.x, hi8.y};
                o[mb] = mfma32<DT>(va, pb, o[mb]);
            }
        }
    };

    // tile kt lives in LDS buffer kt%2
    gload(0, 0);
    lstore(0, 0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; ++kt) {
        const bool more = kt + 1 < ntiles;
        if (more) gload(kt + 1, 0);
        tile(kt, kt & 1);
        if (more) lstore((kt + 1) & 1, 0);
        __syncthreads();
    }

    // ---- epilogue: y (+)= mix * O, optional O and lse
    // every row of the ones-product holds the query's sum; f32 inputs sum in f32
    const float l = SPLIT ? lsum + __shfl_xor(lsum, 32) : lacc[0];
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

// Backward of the inlier pathway (chunked GLA) and of the fused
// RMSNorm / gla_scale / mix epilogue, for gfx950.
//
// No reference kernel: the reference trains through autograd of fla's
// chunk_gla, nn.RMSNorm, the gla_scale product and torch.lerp
// (src/HybridOutlierFactorizedAttentionTrain.py:263-294).  Forward, per head:
//   S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t,  Y_I[t] = q_t S_t
//   N = Y_I * rstd,  Y = (1 - m) gs N + m O
// Gradients, with G the in-chunk inclusive cumsum of g, Q~ = q e^G,
// K~ = k e^-G, K^ = k e^(G_last - G), M = dO V^T and A = Q~ K~^T (both
// masked to key <= query inside the chunk):
//   dN = (1 - m) gs dY,  dO = rstd (dN - N mean(dN N)),  dm = sum_d dY (O - gs N)
//   dH_end(c) = Q~(c+1)^T dO(c+1) + e^(G_last(c+1)) dH_end(c+1)     (reverse scan)
//   dq = e^G (M K~ + dO S_in^T)
//   dk = e^-G (M^T Q~) + e^(G_last - G) (V dH_end^T)
//   dv = A^T dO + K^ dH_end
//   dGamma = q dq - k dk   (gradient of the global cumsum of g), so
//   d log_gamma_t = sum_{s >= t} sum_c a_c dGamma_sc            (a = exp(log_alpha))
//   d log_alpha_c = a_c sum_s dGamma_sc Lambda_s                 (Lambda = cumsum log_gamma)
//   d g_tc        = sum_{s >= t} dGamma_sc                        (general decay)
// Launches:
//   1. gla_bwd_epilogue_kernel  per token: dO (gradient of Y_I), d_mix, mix*dY,
//                               delta = rowsum(mix dY O), gla_scale partials
//   2. gla_state_kernel<BWD>    per chunk: dH^T = dO^T Q~ (shared with the forward)
//   3. gla_bwd_scan_kernel      reverse element-wise scan -> dH_end(c) as hi/lo planes
//   4. gla_bwd_chunk_kernel     per chunk, 4 waves: 2 key-side waves (dk, dv),
//                               2 query-side waves (dq); dGamma reductions
//                               (a factored launch and an element-wise launch for
//                               chunks with a decay range beyond kSafeRange)
//   5. gla_bwd_dlg_kernel       per (batch, head) and 256-token slice: later-chunk suffix of d log_gamma / d g,
//                               d log_alpha and d gla_scale partials
//   6. gla_bwd_param_kernel     per head: d gla_scale, d log_alpha (sum over the batch)
// Every matrix-core product takes bf16 operands; computed operands are hi/lo
// pairs (see split8) and raw f32/f16 inputs are split too, so products track fp32.
//
// This header holds the kernels and their launch sequence.  The launch
// templates are instantiated per (dtype, head dim) in hofa_gla_bwd_inst.hip,
// which the build compiles once per pair so the instantiations build in
// parallel; hofa_gla_bwd.hip holds the C entry point.
#pragma once
#include "hofa_gla_common.h"
#include "hofa_tile.h"

namespace hofa {
namespace glabwd {

using namespace gla;

constexpr int NTB = 256;   // threads of the chunk backward kernel
constexpr int ET = 256;    // tokens per epilogue block
constexpr int kMaxChunks = 4096;


struct GlaBwdK {
    GlaK f;  // forward inputs: q, k, v, lg, la, g, mix, gs with strides; B, H, T, R, nc
    const void *dy, *n, *o;
    const float *rstd;
    const uint16_t *s_in;  // chunk_states, four planes
    void *dq, *dk, *dv, *dlg, *dg, *dla, *dmix, *dgs, *dout;
    float *delta;
    int64_t dy_sb, dy_sh, dy_st, n_sb, n_sh, n_st, o_sb, o_sh, o_st;
    int64_t dq_sb, dq_sh, dq_st, dk_sb, dk_sh, dk_st, dv_sb, dv_sh, dv_st;
    int64_t dlg_sb, dlg_sh, dlg_st, dg_sb, dg_sh, dg_st, dg_sj, dla_sh, dla_sj;
    int64_t dmix_sb, dmix_sh, dmix_st, dgs_sh, dgs_sd, do_sb, do_sh, do_st;
    int dlg_dt, dla_dt, dmix_dt, dgs_dt;
    void *ws_do;        // [B*H][T][D] (dtype of q): gradient of Y_I
    float *ws_dh;       // [B*H][nc][D][J]
    float *ws_gl;       // [B*H][nc][J]
    uint16_t *ds_end;   // [B*H][nc][4][D*J]
    float *dlg_part;    // [B*H][T]
    float *chunk_part;  // [B*H][nc][2J+2]: sum_t dGamma, sum_t dGamma*Lin, e-total, log_gamma total
    float *dgs_part;    // [B*H][ntile][D]
    float *part_la;     // [B*H][J]
    float *part_gs;     // [B*H][D]
    int ntile;
};

template <int DT>
__device__ __forceinline__ void store8(typename Stor<DT>::type *p, const float *x) {
    if constexpr (DT == HOFA_F32) {
        *(f32x4 *)p = f32x4{x[0], x[1], x[2], x[3]};
        *(f32x4 *)(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
    } else {
        *(u32x4 *)p = pack8<DT>(x);
    }
}

// A operand of a k-step of 16 along the permuted index of a C-layout tile
// (entries [16ks + 4hi .. +3] and [16ks + 8 + 4hi .. +3] of an LDS row).
__device__ __forceinline__ u32x4 perm_a(const uint16_t *row, int ks, int hi) {
    const uint16_t *p = row + 16 * ks + 4 * hi;
    const uint2 lo = *(const uint2 *)p, h8 = *(const uint2 *)(p + 8);
    return u32x4{lo.x, lo.y, h8.x, h8.y};
}

// Row of the v-th accumulator entry of a 32x32 C-layout tile.
__device__ __forceinline__ int crow(int v, int hi) { return 8 * (v / 4) + 4 * hi + (v % 4); }

// ---------------------------------------------------------------- 1. epilogue
template <int DT, int D>
__global__ __launch_bounds__(256) void gla_bwd_epilogue_kernel(GlaBwdK a) {
    using in_t = typename Stor<DT>::type;
    constexpr int LPR = D / 8;      // lanes per token row
    constexpr int RPP = 256 / LPR;  // rows per pass
    __shared__ float sP[256][9];
    const int bh = blockIdx.x, tile = blockIdx.y;
    const int H = a.f.H, T = a.f.T;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, slot = tid % LPR, r = tid / LPR, d0 = 8 * slot;
    float gsv[8], part[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        gsv[e] = load_any(a.f.gs, a.f.gs_dt, h * a.f.gs_sh + (d0 + e) * a.f.gs_sd);
        part[e] = 0.f;
    }
    auto group_sum = [](float x) {
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) x += __shfl_xor(x, off);
        return x;
    };
    // The rows of pass p + 1 are loaded while pass p is computed and stored
    // (range-checked buffer loads: rows past T read as zeros).
    const Rows<DT> dyr((const in_t *)a.dy + b * a.dy_sb + h * a.dy_sh, a.dy_st, T);
    const Rows<DT> nr((const in_t *)a.n + b * a.n_sb + h * a.n_sh, a.n_st, T);
    const Rows<DT> orw(a.o ? (const in_t *)a.o + b * a.o_sb + h * a.o_sh : (const in_t *)a.dy, a.o ? a.o_st : 0,
                       a.o ? T : 0);
    struct Pass {
        Raw8<DT> y, n, o;
        float m, rs;
    };
    auto fetch = [&](int t, Pass &p) {
        p.y.load(dyr, t, d0);
        p.n.load(nr, t, d0);
        if (a.o) p.o.load(orw, t, d0);
        p.m = a.f.mix && t < T ? load_any(a.f.mix, a.f.mix_dt, b * a.f.m_sb + h * a.f.m_sh + (int64_t)t * a.f.m_st)
                               : 0.f;
        p.rs = t < T ? a.rstd[(int64_t)bh * T + t] : 0.f;
    };
    Pass cur, nxt;
    fetch(tile * ET + r, cur);
    for (int pass = 0; pass < ET / RPP; ++pass) {
        const int t = tile * ET + pass * RPP + r;
        if (t >= T) break;  // whole row groups leave together
        if (pass + 1 < ET / RPP) fetch(t + RPP, nxt);
        float dy[8], nv[8], ov[8];
        cur.y.get(dy);
        cur.n.get(nv);
        if (a.o) {
            cur.o.get(ov);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) ov[e] = 0.f;
        }
        const float m = cur.m, rs = cur.rs;
        float dn[8], snn = 0.f, syo = 0.f, syn = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float dyi = (1.f - m) * dy[e];
            dn[e] = gsv[e] * dyi;
            part[e] = fmaf(dyi, nv[e], part[e]);
            snn = fmaf(dn[e], nv[e], snn);
            syo = fmaf(dy[e], ov[e], syo);
            syn = fmaf(dy[e], gsv[e] * nv[e], syn);
        }
        snn = group_sum(snn) / (float)D;
        syo = group_sum(syo);
        syn = group_sum(syn);
        float dov[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) dov[e] = rs * (dn[e] - nv[e] * snn);
        store8<DT>((in_t *)a.ws_do + ((int64_t)bh * T + t) * D + d0, dov);
        if (a.dout) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = m * dy[e];
            store8<DT>((in_t *)a.dout + b * a.do_sb + h * a.do_sh + (int64_t)t * a.do_st + d0, x);
        }
        if (slot == 0) {
            if (a.delta) a.delta[(int64_t)bh * T + t] = m * syo;
            if (a.dmix) store_any(a.dmix, a.dmix_dt, b * a.dmix_sb + h * a.dmix_sh + (int64_t)t * a.dmix_st, syo - syn);
        }
        cur = nxt;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) sP[tid][e] = part[e];
    __syncthreads();
    for (int d = tid; d < D; d += 256) {
        float s = 0.f;
        for (int rr = 0; rr < RPP; ++rr) s += sP[rr * LPR + d / 8][d % 8];
        a.dgs_part[((int64_t)bh * a.ntile + tile) * D + d] = s;
    }
}

// ---------------------------------------------------------------- 3. reverse scan
template <int DT, int D, int J>
__global__ __launch_bounds__(kScanRows * J / 4) void gla_bwd_scan_kernel(GlaBwdK a) {
    __shared__ __attribute__((aligned(16))) uint16_t sT[2][2][J * kScanPitch];
    const int bh = blockIdx.x, tid = threadIdx.x;
    const int dvl = tid / (J / 4), j4 = (tid % (J / 4)) * 4;
    const int dv0 = blockIdx.y * kScanRows, dv = dv0 + dvl;
    const int nc = a.f.nc;
    const int64_t base = (int64_t)bh * nc;
    f32x4 X = {0.f, 0.f, 0.f, 0.f};
    constexpr int PF = 4;  // chunks whose loads are in flight together
    for (int c0 = nc - 1; c0 >= 0; c0 -= PF) {
        f32x4 dh[PF], gl[PF];
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int c = max(c0 - u, 0);
            dh[u] = *(const f32x4 *)(a.ws_dh + (base + c) * D * J + dv * J + j4);
            gl[u] = *(const f32x4 *)(a.ws_gl + (base + c) * J + j4);
        }
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int c = c0 - u;
            if (c < 0) break;  // block-uniform
            store_state_tile<DT, D, J>(a.ds_end + (base + c) * 4 * D * J, planes_written<D, J>(4), dv0, dvl, j4, X,
                                       sT[c & 1][0], sT[c & 1][1]);
#pragma unroll
            for (int e = 0; e < 4; ++e) X[e] = fmaf(fast_exp2(gl[u][e] * kLog2e), X[e], dh[u][e]);
        }
    }
}

// ---------------------------------------------------------------- 4. chunk kernel
// FB = false: chunks whose decay range is within kSafeRange (factored
// operands); FB = true: the others (element-wise intra-chunk terms).  Both
// are launched over every chunk and leave at once for the chunks of the other.
//
// Every global load a block needs is issued before its first barrier: the
// decay, the three transposed operand tiles (Q~^T, K~^T, dO^T), each side's
// own rows and the rows of its first loop iteration; a wave whose loop runs
// twice fetches the second iteration's rows during the first.  For D = 64 the
// S^T ([D][J]) hi/lo planes of the exiting (key side) and entering (query
// side) states go to LDS by DMA after the first barrier; S itself is a
// transposing read of the same tiles, so planes 2/3 are neither written nor read.
template <int DT>
__device__ __forceinline__ void raw_op(const Raw8<DT> &r, u32x4 &hi, u32x4 &lo) {
    if constexpr (DT == HOFA_BF16) {
        hi = r.w[0];
        lo = u32x4{0, 0, 0, 0};
    } else {
        float x[8];
        r.get(x);
        split8<OPB>(x, hi, lo);
    }
}

template <int DT, int D, int J, bool GENERAL, bool FB>
__global__ __launch_bounds__(NTB, 2) void gla_bwd_chunk_kernel(GlaBwdK a) {
    using in_t = typename Stor<DT>::type;
    using tile::TileL;
    constexpr int TP = C + 4;             // token pitch of the transposed tiles
    constexpr int JB = (J + 31) / 32;     // 32-row channel blocks
    constexpr int JP = 32 * JB;
    constexpr int KS = J / 16;
    constexpr int DKS = D / 16;
    constexpr int MB = D / 32;
    constexpr bool SPL = kRawSplit<DT>;   // raw f32/f16 inputs are split as well
    constexpr int NO = SPL ? 2 : 1;
    constexpr int DGP = J + 1;             // pitch of the dGamma tile
    constexpr bool SLDS = kStateLds<D, J>;  // state planes staged in LDS (one 64-row tile each)
    static_assert(NTB == tile::NT, "the state DMA splits each tile over four waves");
    __shared__ float sDec[Decay<J, GENERAL>::kFloats];
    __shared__ __attribute__((aligned(16))) uint16_t sQK[2][2][JP * TP];  // [Q~^T | K~^T][hi | lo]
    __shared__ __attribute__((aligned(16))) uint16_t sOt[NO][D * TP];     // dO^T
    // [S_end hi, S_end lo, S_in hi, S_in lo], each S^T [D][J] in the TileL<64> layout
    __shared__ __attribute__((aligned(16))) uint16_t sSt[SLDS ? 4 : 1][SLDS ? TileL<64>::ELEMS : 8];
    static_assert(sizeof(sQK) >= sizeof(float) * C * DGP, "dGamma reuses the operand tiles");
    static_assert(sizeof(sOt) >= sizeof(float) * 2 * NTB, "the channel sums reuse the dO tile");

    const int nc = a.f.nc, H = a.f.H, T = a.f.T, R = a.f.R;
    const int bh = blockIdx.x / nc, c = blockIdx.x % nc;
    const int b = bh / H, h = bh % H, t0 = c * C;
    if ((a.f.unsafe[blockIdx.x] != 0) != FB) return;  // the other launch handles this chunk
    constexpr bool safe = !FB;
    const in_t *qp = (const in_t *)a.f.q + b * a.f.q_sb + h * a.f.q_sh;
    const in_t *kp = (const in_t *)a.f.k + b * a.f.k_sb + h * a.f.k_sh;
    const in_t *vp = (const in_t *)a.f.v + b * a.f.v_sb + h * a.f.v_sh;
    const in_t *dop = (const in_t *)a.ws_do + (int64_t)bh * T * D;
    const Rows<DT> qrows(qp, a.f.q_st, T), krows(kp, a.f.k_st, T), vrows(vp, a.f.v_st, T), drows(dop, D, T);
    const int lane = threadIdx.x & 63, hi = lane >> 5, l32 = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool keyside = w < 2;
    const int own = 32 * (w & 1) + l32;  // key side: key s; query side: query t (chunk-relative)
    const uint16_t *sin = a.s_in + ((int64_t)bh * nc + c) * 4 * D * J;
    const uint16_t *dse = a.ds_end + ((int64_t)bh * nc + c) * 4 * D * J;

    // ---- issue the loads
    DecayStage<J, GENERAL, NTB> dstage;
    TrStage<DT, J, NTB> qst, kst;
    TrStage<DT, D, NTB> ost;
    dstage.issue(a.f, b, h, t0);
    qst.issue(qrows, R, t0);
    kst.issue(krows, R, t0);
    ost.issue(drows, 0, t0);
    Raw8<DT> rA[DKS];  // key side: V row of key own; query side: dO row of query own
    Raw8<DT> rK[KS];   // key side: K row of key own
    Raw8<DT> iA[DKS];  // rows of the current iteration: key side dO, query side V
    Raw8<DT> iQ[KS];   // key side: Q rows of the current iteration
    if (keyside) {
#pragma unroll
        for (int ks = 0; ks < DKS; ++ks) rA[ks].load(vrows, t0 + own, 16 * ks + 8 * hi);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) rK[ks].load(krows, t0 + own, R + 16 * ks + 8 * hi);
#pragma unroll
        for (int ks = 0; ks < DKS; ++ks) iA[ks].load(drows, t0 + own, 16 * ks + 8 * hi);  // first tb = kb
        if constexpr (safe) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) iQ[ks].load(qrows, t0 + own, R + 16 * ks + 8 * hi);
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < DKS; ++ks) rA[ks].load(drows, t0 + own, 16 * ks + 8 * hi);
#pragma unroll
        for (int ks = 0; ks < DKS; ++ks) iA[ks].load(vrows, t0 + l32, 16 * ks + 8 * hi);  // first sb = 0
    }

    // ---- decay, then the transposed operand tiles
    const Decay<J, GENERAL> dec{sDec};
    dstage.commit(a.f, dec);
    qst.template commit<TP, true>(sQK[0][0], sQK[0][1],
                                  [&](int t, int ch) { return fast_exp2(dec.G(t, ch) * kLog2e); });
    kst.template commit<TP, true>(sQK[1][0], sQK[1][1],
                                  [&](int t, int ch) { return fast_exp2(-dec.G(t, ch) * kLog2e); });
    ost.template commit<TP, SPL>(sOt[0], sOt[NO - 1], [](int, int) { return 1.f; });
    if constexpr (JP > J) {
        for (int i = threadIdx.x; i < (JP - J) * TP; i += NTB) {
            sQK[0][0][J * TP + i] = 0;
            sQK[0][1][J * TP + i] = 0;
            sQK[1][0][J * TP + i] = 0;
            sQK[1][1][J * TP + i] = 0;
        }
    }
    __syncthreads();
    // The state planes go to LDS by DMA only now: a barrier waits for every
    // outstanding LDS DMA, so issued earlier they would hold the one above.
    if constexpr (SLDS) {  // S^T planes ([D][J], J columns of a 64-wide tile; the rest zero)
        tile::TileDma<64, J> dm;
        const uint16_t *src[4] = {dse, dse + D * J, sin, sin + D * J};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            dm.init(src[p], J, D, w, lane);
            dm.fetch(sSt[p], 0, w);
        }
    }

    auto qval = [&](int ti, int ch) { return t0 + ti < T ? to_f32<DT>(qp[(int64_t)(t0 + ti) * a.f.q_st + R + ch]) : 0.f; };
    auto kval = [&](int ti, int ch) { return t0 + ti < T ? to_f32<DT>(kp[(int64_t)(t0 + ti) * a.f.k_st + R + ch]) : 0.f; };
    const u32x4 zero4 = {0, 0, 0, 0};
    // K~ / Q~ (= k e^-G / q e^G) at (channel, chunk token) from the staged operands
    auto staged = [&](int which, int ch, int tk) {
        return op_to_f32<OPB>(sQK[which][0][ch * TP + tk]) + op_to_f32<OPB>(sQK[which][1][ch * TP + tk]);
    };
    // A operand S[c][d] (rows c = 32 jb + lane%32, k = d = 16 ks + 8 hi + e) of a
    // state plane pair: a transposing read of the staged S^T tiles, or rows of
    // the [J][D] planes 2/3 in memory
    auto state_row = [&](int which, const uint16_t *g2, int jb, int ks, u32x4 &sh, u32x4 &sl) {
        if constexpr (SLDS) {
            sh = tile::tr_operand_lin<64>(sSt[2 * which], 16 * ks, 32 * jb, lane);
            sl = tile::tr_operand_lin<64>(sSt[2 * which + 1], 16 * ks, 32 * jb, lane);
        } else {
            const int cr = 32 * jb + l32, col = 16 * ks + 8 * hi;
            sh = cr < J ? *(const u32x4 *)(g2 + cr * D + col) : zero4;
            sl = cr < J ? *(const u32x4 *)(g2 + D * J + cr * D + col) : zero4;
        }
    };

    f32x16 acc[JB];  // dk^T (key side) or dq^T (query side): rows = channel, col = token
#pragma unroll
    for (int jb = 0; jb < JB; ++jb)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[jb][v] = 0.f;
    const int tok = own;  // chunk-relative token of this lane's column

    if (keyside) {
        // ================= key side: keys s = 32w + l32
        const int kb = w, s = own, ts = t0 + s;
        f32x16 dvt[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int v = 0; v < 16; ++v) dvt[mb][v] = 0.f;
        u32x4 vh[DKS], vl[DKS];
#pragma unroll
        for (int ks = 0; ks < DKS; ++ks) raw_op<DT>(rA[ks], vh[ks], vl[ks]);
        u32x4 kth[KS], ktl[KS];  // K~ = k e^-G of this key
        if constexpr (safe) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                float x[8];
                rK[ks].get(x);
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] *= fast_exp2(-dec.G(s, 16 * ks + 8 * hi + e) * kLog2e);
                split8<OPB>(x, kth[ks], ktl[ks]);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            if (tb < kb) continue;
            Raw8<DT> nA[DKS], nQ[KS];
            if (tb == 0) {  // wave 0 also has tb = 1: fetch its rows now
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) nA[ks].load(drows, t0 + 32 + l32, 16 * ks + 8 * hi);
                if constexpr (safe) {
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) nQ[ks].load(qrows, t0 + 32 + l32, R + 16 * ks + 8 * hi);
                }
            }
            const int tr = 32 * tb + l32;  // A-operand row (query) of this lane
            f32x16 mt, at;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                mt[v] = 0.f;
                at[v] = 0.f;
            }
            // M[t, s] = sum_d dO[t, d] V[s, d]
#pragma unroll
            for (int ks = 0; ks < DKS; ++ks) {
                u32x4 oh, ol;
                raw_op<DT>(iA[ks], oh, ol);
                mt = mfma32<OPB>(oh, vh[ks], mt);
                if constexpr (SPL) {
                    mt = mfma32<OPB>(oh, vl[ks], mt);
                    mt = mfma32<OPB>(ol, vh[ks], mt);
                }
            }
            // A[t, s] = sum_c q_tc k_sc e^(G_tc - G_sc)
            if constexpr (safe) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    float x[8];
                    iQ[ks].get(x);
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] *= fast_exp2(dec.G(tr, 16 * ks + 8 * hi + e) * kLog2e);
                    u32x4 qh, ql;
                    split8<OPB>(x, qh, ql);
                    at = mfma32<OPB>(qh, kth[ks], at);
                    at = mfma32<OPB>(qh, ktl[ks], at);
                    at = mfma32<OPB>(ql, kth[ks], at);
                }
            } else {
                for (int ch = 0; ch < J; ++ch) {
                    const float kv = kval(s, ch), gs_ = dec.G(s, ch);
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int ti = 32 * tb + crow(v, hi);
                        if (ti >= s) at[v] = fmaf(qval(ti, ch) * kv, fast_exp2((dec.G(ti, ch) - gs_) * kLog2e), at[v]);
                    }
                }
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                if (32 * tb + crow(v, hi) < s) {
                    mt[v] = 0.f;
                    at[v] = 0.f;
                }
            }
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const int ks4 = 2 * tb + k2;
                u32x4 ah, al;
                split8v<OPB>(at, 8 * k2, ah, al);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const int ro = (32 * mb + l32) * TP;
                    const u32x4 oa = perm_a(&sOt[0][ro], ks4, hi);
                    dvt[mb] = mfma32<OPB>(oa, ah, dvt[mb]);
                    dvt[mb] = mfma32<OPB>(oa, al, dvt[mb]);
                    if constexpr (SPL) dvt[mb] = mfma32<OPB>(perm_a(&sOt[NO - 1][ro], ks4, hi), ah, dvt[mb]);
                }
                if constexpr (safe) {
                    u32x4 mh, ml;
                    split8v<OPB>(mt, 8 * k2, mh, ml);
#pragma unroll
                    for (int jb = 0; jb < JB; ++jb) {
                        const int ro = (32 * jb + l32) * TP;
                        const u32x4 qa = perm_a(&sQK[0][0][ro], ks4, hi), qal = perm_a(&sQK[0][1][ro], ks4, hi);
                        acc[jb] = mfma32<OPB>(qa, mh, acc[jb]);
                        acc[jb] = mfma32<OPB>(qa, ml, acc[jb]);
                        acc[jb] = mfma32<OPB>(qal, mh, acc[jb]);
                    }
                }
            }
            if constexpr (!safe) {  // dk_sc += sum_t M[t, s] q_tc e^(G_tc - G_sc) over the tile's rows (both lane halves)
                f32x16 mo;
#pragma unroll
                for (int v = 0; v < 16; ++v) mo[v] = __shfl_xor(mt[v], 32);
#pragma unroll
                for (int jb = 0; jb < JB; ++jb)
#pragma unroll
                    for (int vv = 0; vv < 16; ++vv) {
                        const int ch = 32 * jb + crow(vv, hi);
                        if (ch >= J) continue;
                        const float gsc = dec.G(s, ch);
                        float x = 0.f;
                        for (int v = 0; v < 16; ++v) {
                            const int ta = 32 * tb + crow(v, hi), tbb = 32 * tb + crow(v, 1 - hi);
                            if (ta >= s) x = fmaf(mt[v] * qval(ta, ch), fast_exp2((dec.G(ta, ch) - gsc) * kLog2e), x);
                            if (tbb >= s) x = fmaf(mo[v] * qval(tbb, ch), fast_exp2((dec.G(tbb, ch) - gsc) * kLog2e), x);
                        }
                        acc[jb][vv] += x;
                    }
            }
            if (tb == 0) {
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) iA[ks] = nA[ks];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) iQ[ks] = nQ[ks];
            }
        }
        if constexpr (SLDS) tile::wait_vmem();
        __syncthreads();  // the state tiles are complete (the query side waits at its own barrier)
        in_t *dkr = (in_t *)a.dk + b * a.dk_sb + h * a.dk_sh + (int64_t)ts * a.dk_st + R;
        in_t *dvr = (in_t *)a.dv + b * a.dv_sb + h * a.dv_sh + (int64_t)ts * a.dv_st;
        // dk = e^-G (intra + e^G_last X) (factored) or intra + e^(G_last - G) X (element-wise),
        // X = sum_d dH_end[c, d] V[s, d]; acc then holds this key's part of dGamma, -k dk
#pragma unroll
        for (int jb = 0; jb < JB; ++jb) {
            f32x16 x = {};
            if (c < nc - 1) {
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) {
                    u32x4 sh, sl;
                    state_row(0, dse + 2 * D * J, jb, ks, sh, sl);
                    x = mfma32<OPB>(sh, vh[ks], x);
                    x = mfma32<OPB>(sl, vh[ks], x);
                    if constexpr (SPL) x = mfma32<OPB>(sh, vl[ks], x);
                }
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int ch0 = 32 * jb + 8 * g + 4 * hi;
                if (ch0 >= J) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[jb][4 * g + e] = 0.f;
                    continue;
                }
                float dk4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int v = 4 * g + e, ch = ch0 + e;
                    if constexpr (safe) {
                        const float y = fmaf(fast_exp2(dec.last(ch) * kLog2e), x[v], acc[jb][v]);
                        dk4[e] = y * fast_exp2(-dec.G(s, ch) * kLog2e);
                        acc[jb][v] = -staged(1, ch, s) * y;
                    } else {
                        dk4[e] = fmaf(fast_exp2((dec.last(ch) - dec.G(s, ch)) * kLog2e), x[v], acc[jb][v]);
                        acc[jb][v] = -kval(s, ch) * dk4[e];
                    }
                }
                if (ts < T) store4<DT>(dkr + ch0, dk4[0], dk4[1], dk4[2], dk4[3]);
            }
        }
        if (c < nc - 1) {  // dv^T[d, s] += sum_c dH_end^T[d, c] K^[s, c]
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                float x[8];
                rK[ks].get(x);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int ch = 16 * ks + 8 * hi + e;
                    x[e] *= fast_exp2((dec.last(ch) - dec.G(s, ch)) * kLog2e);
                }
                u32x4 kh, kl;
                split8<OPB>(x, kh, kl);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    u32x4 sh, sl;
                    if constexpr (SLDS) {  // A[d, c] = S_end^T rows of the staged tiles
                        const int o = TileL<64>::off(32 * mb + l32, 16 * ks + 8 * hi);
                        sh = *(const u32x4 *)&sSt[0][o];
                        sl = *(const u32x4 *)&sSt[1][o];
                    } else {
                        const int off = (32 * mb + l32) * J + 16 * ks + 8 * hi;
                        sh = *(const u32x4 *)(dse + off);
                        sl = *(const u32x4 *)(dse + D * J + off);
                    }
                    dvt[mb] = mfma32<OPB>(sh, kh, dvt[mb]);
                    dvt[mb] = mfma32<OPB>(sh, kl, dvt[mb]);
                    dvt[mb] = mfma32<OPB>(sl, kh, dvt[mb]);
                }
            }
        }
        if (ts < T) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    store4<DT>(dvr + 32 * mb + 8 * g + 4 * hi, dvt[mb][4 * g], dvt[mb][4 * g + 1], dvt[mb][4 * g + 2],
                               dvt[mb][4 * g + 3]);
        }
    } else {
        // ================= query side: queries t = 32(w-2) + l32
        const int qb = w - 2, t = own, tq = t0 + t;
        u32x4 dh[DKS], dl[DKS];
#pragma unroll
        for (int ks = 0; ks < DKS; ++ks) raw_op<DT>(rA[ks], dh[ks], dl[ks]);
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
            if (sb > qb) break;
            Raw8<DT> nA[DKS];
            if (sb == 0 && qb == 1) {  // fetch the second key block's rows now
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) nA[ks].load(vrows, t0 + 32 + l32, 16 * ks + 8 * hi);
            }
            f32x16 mt;
#pragma unroll
            for (int v = 0; v < 16; ++v) mt[v] = 0.f;
            // M^T[s, t] = sum_d V[s, d] dO[t, d]
#pragma unroll
            for (int ks = 0; ks < DKS; ++ks) {
                u32x4 va, vla;
                raw_op<DT>(iA[ks], va, vla);
                mt = mfma32<OPB>(va, dh[ks], mt);
                if constexpr (SPL) {
                    mt = mfma32<OPB>(va, dl[ks], mt);
                    mt = mfma32<OPB>(vla, dh[ks], mt);
                }
            }
#pragma unroll
            for (int v = 0; v < 16; ++v)
                if (32 * sb + crow(v, hi) > t) mt[v] = 0.f;
            if constexpr (safe) {
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    const int ks4 = 2 * sb + k2;
                    u32x4 mh, ml;
                    split8v<OPB>(mt, 8 * k2, mh, ml);
#pragma unroll
                    for (int jb = 0; jb < JB; ++jb) {
                        const int ro = (32 * jb + l32) * TP;
                        const u32x4 ka = perm_a(&sQK[1][0][ro], ks4, hi), kal = perm_a(&sQK[1][1][ro], ks4, hi);
                        acc[jb] = mfma32<OPB>(ka, mh, acc[jb]);
                        acc[jb] = mfma32<OPB>(ka, ml, acc[jb]);
                        acc[jb] = mfma32<OPB>(kal, mh, acc[jb]);
                    }
                }
            } else {  // dq_tc += sum_s M[t, s] k_sc e^(G_tc - G_sc)
                f32x16 mo;
#pragma unroll
                for (int v = 0; v < 16; ++v) mo[v] = __shfl_xor(mt[v], 32);
#pragma unroll
                for (int jb = 0; jb < JB; ++jb)
#pragma unroll
                    for (int vv = 0; vv < 16; ++vv) {
                        const int ch = 32 * jb + crow(vv, hi);
                        if (ch >= J) continue;
                        const float gtc = dec.G(t, ch);
                        float x = 0.f;
                        for (int v = 0; v < 16; ++v) {
                            const int sa = 32 * sb + crow(v, hi), sbb = 32 * sb + crow(v, 1 - hi);
                            if (sa <= t) x = fmaf(mt[v] * kval(sa, ch), fast_exp2((gtc - dec.G(sa, ch)) * kLog2e), x);
                            if (sbb <= t) x = fmaf(mo[v] * kval(sbb, ch), fast_exp2((gtc - dec.G(sbb, ch)) * kLog2e), x);
                        }
                        acc[jb][vv] += x;
                    }
            }
            if (sb == 0 && qb == 1) {
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) iA[ks] = nA[ks];
            }
        }
        if constexpr (SLDS) tile::wait_vmem();
        __syncthreads();  // pairs with the key side's barrier: the state tiles are complete
        // dq^T[c, t] (+)= e^G_tc (sum_d S_in[c, d] dO[t, d])
#pragma unroll
        for (int jb = 0; jb < JB; ++jb) {
            f32x16 x;
#pragma unroll
            for (int v = 0; v < 16; ++v) x[v] = 0.f;
            if (c > 0) {
#pragma unroll
                for (int ks = 0; ks < DKS; ++ks) {
                    u32x4 sh, sl;
                    state_row(1, sin + 2 * D * J, jb, ks, sh, sl);
                    x = mfma32<OPB>(sh, dh[ks], x);
                    x = mfma32<OPB>(sl, dh[ks], x);
                    if constexpr (SPL) x = mfma32<OPB>(sh, dl[ks], x);
                }
            }
            // dq = e^G (intra + X) (factored) or intra + e^G X (element-wise); acc then holds q dq
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int ch0 = 32 * jb + 8 * g + 4 * hi;
                if (ch0 >= J) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[jb][4 * g + e] = 0.f;
                    continue;
                }
                float dq4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int v = 4 * g + e, ch = ch0 + e;
                    const float eg = fast_exp2(dec.G(t, ch) * kLog2e);
                    if constexpr (safe) {
                        const float y = acc[jb][v] + x[v];
                        dq4[e] = eg * y;
                        acc[jb][v] = staged(0, ch, t) * y;
                    } else {
                        dq4[e] = fmaf(eg, x[v], acc[jb][v]);
                        acc[jb][v] = qval(t, ch) * dq4[e];
                    }
                }
                if (tq < T)
                    store4<DT>((in_t *)a.dq + b * a.dq_sb + h * a.dq_sh + (int64_t)tq * a.dq_st + R + ch0, dq4[0], dq4[1],
                               dq4[2], dq4[3]);
            }
        }
    }

    // ---- dGamma = q dq - k dk in LDS (reusing the operand tiles)
    __syncthreads();
    float *sDG = (float *)&sQK[0][0][0];
    if (w >= 2) {
#pragma unroll
        for (int jb = 0; jb < JB; ++jb)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int ch = 32 * jb + crow(v, hi);
                if (ch < J) sDG[tok * DGP + ch] = acc[jb][v];
            }
    }
    __syncthreads();
    if (w < 2) {
#pragma unroll
        for (int jb = 0; jb < JB; ++jb)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int ch = 32 * jb + crow(v, hi);
                if (ch < J) sDG[tok * DGP + ch] += acc[jb][v];
            }
    }
    __syncthreads();
    float *cp = a.chunk_part + ((int64_t)bh * nc + c) * (2 * J + 2);
    const int tid = threadIdx.x;
    if constexpr (!GENERAL) {
        const float *sLam = sDec, *sAl = sDec + C;
        if (w == 0) {  // d log_gamma partial: suffix over the chunk's tokens of sum_c alpha_c dGamma
            float e = 0.f;
            for (int ch = 0; ch < J; ++ch) e = fmaf(sAl[ch], sDG[lane * DGP + ch], e);
            const float incl = wave_incl_scan(e);
            const float total = __shfl(incl, 63);
            if (t0 + lane < T) a.dlg_part[(int64_t)bh * T + t0 + lane] = total - incl + e;
            if (lane == 0) {
                cp[2 * J] = total;
                cp[2 * J + 1] = sLam[C - 1];
            }
        }
        // per channel: sum_t dGamma and sum_t dGamma Lambda_t, NSEG token segments per channel
        constexpr int NSEG = NTB / J;
        float *red = (float *)&sOt[0][0];
        const int ch = tid % J, seg = tid / J;
        float ed = 0.f, f = 0.f;
        if (seg < NSEG) {
            for (int t = seg; t < C; t += NSEG) {
                const float x = sDG[t * DGP + ch];
                ed += x;
                f = fmaf(x, sLam[t], f);
            }
        }
        red[tid] = ed;
        red[NTB + tid] = f;
        __syncthreads();
        if (tid < J) {
            float se = 0.f, sf = 0.f;
#pragma unroll
            for (int sg = 0; sg < NSEG; ++sg) {
                se += red[sg * J + tid];
                sf += red[NTB + sg * J + tid];
            }
            cp[tid] = se;
            cp[J + tid] = sf;
        }
    } else {
        // d g: suffix over the chunk's tokens per channel (lane = token), written back, then stored by rows
        constexpr int NW = NTB / 64;
        for (int ch = w; ch < J; ch += NW) {
            const float x = sDG[lane * DGP + ch];
            const float incl = wave_incl_scan(x);
            const float total = __shfl(incl, 63);
            sDG[lane * DGP + ch] = total - incl + x;
            if (lane == 0) cp[ch] = total;
        }
        __syncthreads();
        float *dg = (float *)a.dg + b * a.dg_sb + h * a.dg_sh;
        for (int idx = tid; idx < C * J; idx += NTB) {
            const int t = idx / J, ch = idx % J;
            if (t0 + t < T) dg[(int64_t)(t0 + t) * a.dg_st + ch * a.dg_sj] = sDG[t * DGP + ch];
        }
    }
}

// ---------------------------------------------------------------- 5. per-head suffix and partials
// Grid (B*H, kDlgTokens-token slices + 2).  A slice block adds the
// later-chunk suffix to d log_gamma (or d g) of its tokens; block NSL
// reduces this head's d log_alpha partials over chunks, block NSL + 1 its
// d gla_scale partials over token tiles.  Every block has one short chain of
// loads (96 heads of one block each left the GPU waiting on four in a row).
constexpr int kDlgTokens = 256;  // tokens per slice block
constexpr int kDlgChunks = kDlgTokens / C;

template <int D, int J, bool GENERAL>
__global__ __launch_bounds__(256) void gla_bwd_dlg_kernel(GlaBwdK a) {
    __shared__ float sLst[kMaxChunks];            // cumsum of log_gamma before the chunk (d log_alpha block)
    __shared__ float sSfx[kDlgChunks][GENERAL ? J : 1];  // suffix over later chunks, per chunk of the slice
    __shared__ float sRed[256];
    constexpr int CPS = 2 * J + 2;
    const int bh = blockIdx.x, H = a.f.H, T = a.f.T, nc = a.f.nc;
    const int b = bh / H, h = bh % H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nsl = (T + kDlgTokens - 1) / kDlgTokens;
    const int y = blockIdx.y;
    const float *cp = a.chunk_part + (int64_t)bh * nc * CPS;
    if (y < nsl) {
        const int c_lo = y * kDlgChunks, c_hi = min(nc, c_lo + kDlgChunks);
        if constexpr (!GENERAL) {
            // sum of e over the chunks past the slice, then the slice's own suffixes
            float part = 0.f;
            for (int c = c_hi + tid; c < nc; c += 256) part += cp[(int64_t)c * CPS + 2 * J];
            part = wave_sum(part);
            if (lane == 0) sRed[w] = part;
            __syncthreads();
            if (tid == 0) {
                float carry = sRed[0] + sRed[1] + sRed[2] + sRed[3];
                for (int c = c_hi - 1; c >= c_lo; --c) {
                    sSfx[c - c_lo][0] = carry;
                    carry += cp[(int64_t)c * CPS + 2 * J];
                }
            }
            __syncthreads();
            const int t = y * kDlgTokens + tid;
            if (t < T)
                store_any(a.dlg, a.dlg_dt, b * a.dlg_sb + h * a.dlg_sh + (int64_t)t * a.dlg_st,
                          a.dlg_part[(int64_t)bh * T + t] + sSfx[t / C - c_lo][0]);
        } else {
            // per channel: sum over the chunks past the slice, then the slice's own suffixes
            for (int ch = tid; ch < J; ch += 256) {
                float carry = 0.f;
                for (int c = c_hi; c < nc; ++c) carry += cp[(int64_t)c * CPS + ch];
                for (int c = c_hi - 1; c >= c_lo; --c) {
                    sSfx[c - c_lo][ch] = carry;
                    carry += cp[(int64_t)c * CPS + ch];
                }
            }
            __syncthreads();
            float *dg = (float *)a.dg + b * a.dg_sb + h * a.dg_sh;
            const int t0 = y * kDlgTokens, nt = min(kDlgTokens, T - t0);
            for (int i = tid; i < nt * J; i += 256) {
                const int t = t0 + i / J, ch = i % J;
                dg[(int64_t)t * a.dg_st + ch * a.dg_sj] += sSfx[t / C - c_lo][ch];
            }
        }
    } else if (y == nsl) {
        // sum_c (Lambda_start(c) sum_t dGamma + sum_t dGamma Lambda_in), channel-parallel
        if (GENERAL || !a.dla) return;
        if (w == 0) {  // exclusive prefix of the per-chunk log_gamma totals
            float carry = 0.f;
            for (int c0 = 0; c0 < nc; c0 += 64) {
                const int c = c0 + lane;
                const float l = c < nc ? cp[(int64_t)c * CPS + 2 * J + 1] : 0.f;
                const float x = wave_incl_scan(l);
                if (c < nc) sLst[c] = carry + x - l;
                carry += __shfl(x, 63);
            }
        }
        __syncthreads();
        constexpr int NSEG = 256 / J;
        const int ch = tid % J, seg = tid / J;
        float acc = 0.f;
        if (seg < NSEG)
            for (int c = seg; c < nc; c += NSEG) {
                const float *p = cp + (int64_t)c * CPS;
                acc = fmaf(sLst[c], p[ch], acc + p[J + ch]);
            }
        sRed[tid] = acc;
        __syncthreads();
        if (tid < J) {
            float t = 0.f;
            for (int sg = 0; sg < NSEG; ++sg) t += sRed[sg * J + tid];
            a.part_la[(int64_t)bh * J + tid] = t;
        }
    } else {
        for (int d = tid; d < D; d += 256) {
            float s = 0.f;
            for (int tile = 0; tile < a.ntile; ++tile) s += a.dgs_part[((int64_t)bh * a.ntile + tile) * D + d];
            a.part_gs[(int64_t)bh * D + d] = s;
        }
    }
}

// ---------------------------------------------------------------- 6. per-head parameters
template <int D, int J, bool GENERAL>
__global__ __launch_bounds__(256) void gla_bwd_param_kernel(GlaBwdK a) {
    const int h = blockIdx.x, H = a.f.H, B = a.f.B;
    for (int d = threadIdx.x; d < D; d += 256) {
        float s = 0.f;
        for (int b = 0; b < B; ++b) s += a.part_gs[(int64_t)(b * H + h) * D + d];
        store_any(a.dgs, a.dgs_dt, h * a.dgs_sh + d * a.dgs_sd, s);
    }
    if constexpr (!GENERAL) {
        if (!a.dla) return;
        for (int ch = threadIdx.x; ch < J; ch += 256) {
            float s = 0.f;
            for (int b = 0; b < B; ++b) s += a.part_la[(int64_t)(b * H + h) * J + ch];
            const float alpha = expf(load_any(a.f.la, a.f.la_dt, h * a.f.la_sh + ch * a.f.la_sj));
            store_any(a.dla, a.dla_dt, h * a.dla_sh + ch * a.dla_sj, alpha * s);
        }
    }
}

template <int DT, int D, int J, bool GEN>
void launch(const GlaBwdK &k, hipStream_t s) {
    const int nbh = k.f.B * k.f.H;
    hipLaunchKernelGGL((gla_bwd_epilogue_kernel<DT, D>), dim3(nbh, k.ntile), dim3(256), 0, s, k);
    GlaK fk = k.f;  // dH^T = dO^T (q e^G): key operand q at column R, value operand dO
    fk.k = k.f.q;
    fk.k_sb = k.f.q_sb; fk.k_sh = k.f.q_sh; fk.k_st = k.f.q_st;
    fk.key_col0 = k.f.R;
    fk.v = k.ws_do;
    fk.v_sb = (int64_t)k.f.H * k.f.T * D; fk.v_sh = (int64_t)k.f.T * D; fk.v_st = D;
    fk.ws_ds = k.ws_dh;
    fk.ws_gl = k.ws_gl;
    hipLaunchKernelGGL((gla_state_kernel<DT, D, J, GEN, true>), dim3(nbh * k.f.nc), dim3(kStateThreads), 0, s, fk);
    hipLaunchKernelGGL((gla_bwd_scan_kernel<DT, D, J>), dim3(nbh, D / kScanRows), dim3(kScanRows * J / 4), 0, s, k);
    hipLaunchKernelGGL((gla_bwd_chunk_kernel<DT, D, J, GEN, false>), dim3(nbh * k.f.nc), dim3(NTB), 0, s, k);
    hipLaunchKernelGGL((gla_bwd_chunk_kernel<DT, D, J, GEN, true>), dim3(nbh * k.f.nc), dim3(NTB), 0, s, k);
    hipLaunchKernelGGL((gla_bwd_dlg_kernel<D, J, GEN>), dim3(nbh, (k.f.T + kDlgTokens - 1) / kDlgTokens + 2),
                       dim3(256), 0, s, k);
    hipLaunchKernelGGL((gla_bwd_param_kernel<D, J, GEN>), dim3(k.f.H), dim3(256), 0, s, k);
}

// Every launch of one backward pass for head dim D; J is the inlier width.
template <int DT, int D, bool GEN>
int launch_d(const GlaBwdK &k, int J, hipStream_t s) {
    if constexpr (D == 64) {
        if (J == 48) launch<DT, 64, 48, GEN>(k, s);
        else if (J == 32) launch<DT, 64, 32, GEN>(k, s);
        else if (J == 64) launch<DT, 64, 64, GEN>(k, s);
        else return HOFA_EUNSUPPORTED;
    } else {
        if (J == 112) launch<DT, 128, 112, GEN>(k, s);
        else if (J == 96) launch<DT, 128, 96, GEN>(k, s);
        else if (J == 64) launch<DT, 128, 64, GEN>(k, s);
        else if (J == 128) launch<DT, 128, 128, GEN>(k, s);
        else return HOFA_EUNSUPPORTED;
    }
    return HOFA_OK;
}

#define HOFA_GLA_BWD_FOR_EACH(X)                                     \
    X(HOFA_F32, 64) X(HOFA_F32, 128) X(HOFA_BF16, 64) X(HOFA_BF16, 128) \
    X(HOFA_F16, 64) X(HOFA_F16, 128)

}  // namespace glabwd
}  // namespace hofa

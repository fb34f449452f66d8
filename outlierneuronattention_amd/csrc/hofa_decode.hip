// Split-K HOFA decode for gfx950: two launches per token.
//
// Replaces fused_hofa_decode and its Triton kernels
// (src/hofa_decode_triton.py:173-239 split, :242-340 reduce, host :342-476).
//
// 1. stream kernel, grid B*H + B*H*n_split, 256 threads.  The first B*H
//    blocks apply the GLA update S' = gamma (.) S + k_I^T v to one head's
//    [J, D] fp32 state (float4 rows) and write y_I = q_I S'.  Every other
//    block (head, split) runs an online softmax over cache rows
//    [split*tps, (split+1)*tps) of one head.
//    Each wave owns a quarter of the range; rows are fetched as 16-byte buffer
//    loads (a tile of TT tokens is eight V vectors per lane, LPR lanes per V
//    row, plus 8R/D K vectors per lane, KL lanes per K row) and the next tile
//    is in flight while the current one is consumed.  Rows at or beyond the
//    valid length read as zero through the buffer range check and get a -inf
//    score.  The four waves merge in LDS and the block writes one partial
//    (m, l, acc[D]) in the base-2 log domain.
//    The state block also finishes the inlier side,
//    z = (1 - mix) * RMSNorm(y_I) * norm_w, and stores z and mix.
// 2. merge kernel, grid B*H, one wave per head: loads the partials in batches
//    issued before use, merges them by log-sum-exp and writes
//    y = mix * y_O + z.
// The kernel boundary orders the partial writes before the merge's reads, so
// no device-scope fence or counter is needed and the workspace carries no
// state between calls.
#include <mutex>

#include "hofa_common.h"

namespace hofa {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSplit = 64;  // partials merged per head (one per lane of the merge wave)
constexpr int kPlanMaxSplit = 48;  // the automatic plan's cap
constexpr float kRefTau = 16.f;    // a split's softmax reference moves only for scores beyond it by more (log2 units)
constexpr int kBufFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)
constexpr int kLoadNT = 2;             // non-temporal hint for streamed cache rows

struct DecodeKArgs {
    const void *q, *k, *v, *cache_k, *cache_v;
    const float *state_in;
    float *state_out;
    const void *log_gamma, *mix, *norm_w, *log_alpha;
    void *y;
    const int32_t *seq_len_dev;
    float *ws_acc;  // [B*H][n_split][D] partial numerators
    float *ws_ml;   // [B*H][n_split][2] partial (max, denominator), base-2 domain
    float *ws_z;    // [B*H][D + 4] inlier contribution and mix
    int64_t q_sb, q_sh, q_sd, k_sb, k_sh, k_sd, v_sb, v_sh, v_sd;
    int64_t ck_sb, ck_sh, ck_sl, cv_sb, cv_sh, cv_sl;
    int64_t st_sb, st_sh, so_sb, so_sh;
    int64_t lg_sb, lg_sh, mg_sb, mg_sh, nw_sh, nw_sd, la_sh, la_sj;
    int64_t y_sb, y_sh, y_sd;
    int lg_dt, mg_dt, nw_dt, la_dt;
    int B, H;
    int seq_len, cache_len;
    int n_split, tps;
    float qscale;  // sm_scale * log2(e): scores live in the base-2 domain
    float eps;
    int nslot;     // partials per head: n_split, plus the new token's with the in-kernel prologue
    // in-kernel prologue (hofa_decode_fused): gates, RoPE and cache append of the new token
    const void *gate_w, *gate_b, *mix_w, *mix_b, *fixed_mix, *rcos, *rsin;
    int rope, rope_dt, rope_rows;
};

template <int DT, int D>
struct Geometry {
    static constexpr int EPV = Vec<DT>::epv;  // elements per 16-byte vector
    static constexpr int LPR = D / EPV;       // lanes per V row
    static constexpr int TT = 64 * 8 / LPR;   // tokens per tile
};

__device__ __forceinline__ int current_len(const DecodeKArgs &a) {
    return a.seq_len_dev ? min(*a.seq_len_dev, a.cache_len) : a.seq_len;
}

template <int DT>
__device__ __forceinline__ float rnd_st(float v) {
    return to_f32<DT>(from_f32<DT>(v));
}

// One rotated element x' = x cos + rotate_half(x) sin (partner = the element
// half a rotation away, lower = the element sits in the first half).  16-bit
// tables round each product as a 16-bit module computes it; f32 tables round
// once.  The same expression as hofa_decode_prologue, so both paths agree.
template <int DT>
__device__ __forceinline__ float rope1(float x, float partner, bool lower, float c, float s, int rope_dt) {
    const float sg = lower ? -1.f : 1.f;
    if (rope_dt == HOFA_F32) return rnd_st<DT>(x * c + sg * partner * s);
    return rnd_st<DT>(rnd_st<DT>(x * c) + rnd_st<DT>(sg * partner * s));
}

// GLA state update of one head; (1 - mix) * RMSNorm(y_I) * norm_w and mix go to the workspace.
template <int DT, int D, int R>
__device__ void state_block(const DecodeKArgs &a, int bh) {
    using st = typename Stor<DT>::type;
    constexpr int J = D - R;
    constexpr int DV4 = D / 4;
    constexpr int RG = kThreads / DV4;  // state rows per pass
    constexpr int NPASS = (J + RG - 1) / RG;
    __shared__ float s_v[D], s_k[J], s_q[J], s_g[J];
    __shared__ float s_red[RG * D];
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x;
    const int d4 = (tid % DV4) * 4, jr = tid / DV4;
    const float *sin = a.state_in + b * a.st_sb + h * a.st_sh;
    f32x4 srow[NPASS];
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
        const int j = jr + i * RG;
        srow[i] = j < J ? *(const f32x4 *)(sin + j * D + d4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const st *qp = (const st *)a.q + b * a.q_sb + h * a.q_sh;
    const st *kp = (const st *)a.k + b * a.k_sb + h * a.k_sh;
    const st *vp = (const st *)a.v + b * a.v_sb + h * a.v_sh;
    for (int i = tid; i < D; i += kThreads) s_v[i] = to_f32<DT>(vp[i * a.v_sd]);
    const float lg = load_any(a.log_gamma, a.lg_dt, b * a.lg_sb + h * a.lg_sh);
    for (int i = tid; i < J; i += kThreads) {
        s_k[i] = to_f32<DT>(kp[(R + i) * a.k_sd]);
        s_q[i] = to_f32<DT>(qp[(R + i) * a.q_sd]);
        float e = lg;
        if (a.log_alpha) e = lg * expf(load_any(a.log_alpha, a.la_dt, h * a.la_sh + i * a.la_sj));
        s_g[i] = expf(e);
    }
    __syncthreads();
    float *sout = a.state_out + b * a.so_sb + h * a.so_sh;
    const f32x4 vv = {s_v[d4], s_v[d4 + 1], s_v[d4 + 2], s_v[d4 + 3]};
    f32x4 yp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
        const int j = jr + i * RG;
        if (j < J) {
            const f32x4 sn = s_g[j] * srow[i] + s_k[j] * vv;
            *(f32x4 *)(sout + j * D + d4) = sn;
            yp += s_q[j] * sn;
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) s_red[jr * D + d4 + c] = yp[c];
    __syncthreads();
    // Finish the inlier side: z = (1 - mix) * RMSNorm(y_I; eps) * norm_w.
    float y = 0.f;
    if (tid < D) {
#pragma unroll
        for (int r = 0; r < RG; ++r) y += s_red[r * D + tid];
    }
    float ss = wave_sum(y * y);  // D <= 128: waves 0 and 1 hold y
    __shared__ float s_ss[kWaves];
    if ((tid & 63) == 0) s_ss[tid >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) ss += s_ss[w];
    const float mix = load_any(a.mix, a.mg_dt, b * a.mg_sb + h * a.mg_sh);
    float *z = a.ws_z + bh * (D + 4);
    if (tid < D) {
        const float nw = load_any(a.norm_w, a.nw_dt, h * a.nw_sh + tid * a.nw_sd);
        z[tid] = (1.f - mix) * (y * rsqrtf(ss / (float)D + a.eps) * nw);
    }
    if (tid == 0) z[D] = mix;
}

// The state block with the prologue of the new token folded in: gates from the
// pre-RoPE q/k, RoPE of the outlier channels at pos = seq_len - 1, the cache
// append of that row, the token's own softmax partial (m = q.k * scale, l = 1,
// acc = v) as partial n_split, then the GLA update and inlier epilogue.
template <int DT, int D, int R>
__device__ void state_block_pro(const DecodeKArgs &a, int bh) {
    using st = typename Stor<DT>::type;
    constexpr int J = D - R;
    constexpr int DV4 = D / 4;
    constexpr int RG = kThreads / DV4;  // state rows per pass
    constexpr int NPASS = (J + RG - 1) / RG;
    static_assert(R <= 64, "the token's outlier score is one wave's sum");
    __shared__ float s_q[D], s_k[D], s_v[D], s_g[J];
    __shared__ float s_red[RG * D];
    __shared__ float s_gate[2];  // log_gamma, mix
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int d4 = (tid % DV4) * 4, jr = tid / DV4;
    const int pos = max(current_len(a) - 1, 0);
    const float *sin = a.state_in + b * a.st_sb + h * a.st_sh;
    f32x4 srow[NPASS];
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
        const int j = jr + i * RG;
        srow[i] = j < J ? *(const f32x4 *)(sin + j * D + d4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const st *qp = (const st *)a.q + b * a.q_sb + h * a.q_sh;
    const st *kp = (const st *)a.k + b * a.k_sb + h * a.k_sh;
    const st *vp = (const st *)a.v + b * a.v_sb + h * a.v_sh;
    for (int i = tid; i < D; i += kThreads) {
        s_q[i] = to_f32<DT>(qp[i * a.q_sd]);
        s_k[i] = to_f32<DT>(kp[i * a.k_sd]);
        s_v[i] = to_f32<DT>(vp[i * a.v_sd]);
    }
    __syncthreads();
    if (tid < 64) {  // gate and mix logits on the pre-RoPE q, k, rounded as the module's 16-bit ops
        const st *gw = (const st *)a.gate_w + h * 2 * D;
        const st *mw = a.mix_w ? (const st *)a.mix_w + h * 2 * D : nullptr;
        float gq = 0.f, gk = 0.f, mq = 0.f, mk = 0.f;
        for (int d = lane; d < D; d += 64) {
            gq = fmaf(s_q[d], to_f32<DT>(gw[d]), gq);
            gk = fmaf(s_k[d], to_f32<DT>(gw[D + d]), gk);
            if (mw) {
                mq = fmaf(s_q[d], to_f32<DT>(mw[d]), mq);
                mk = fmaf(s_k[d], to_f32<DT>(mw[D + d]), mk);
            }
        }
        gq = wave_sum(gq);
        gk = wave_sum(gk);
        mq = wave_sum(mq);
        mk = wave_sum(mk);
        if (lane == 0) {  // each einsum rounded, then their sum, then the sum with the bias
            const float gl = rnd_st<DT>(rnd_st<DT>(rnd_st<DT>(gq) + rnd_st<DT>(gk)) +
                                        to_f32<DT>(((const st *)a.gate_b)[h]));
            const float ng = -gl;
            s_gate[0] = rnd_st<DT>(fminf(ng, 0.f) - log1pf(expf(-fabsf(ng))));
            const float ml = mw ? rnd_st<DT>(rnd_st<DT>(rnd_st<DT>(mq) + rnd_st<DT>(mk)) +
                                             to_f32<DT>(((const st *)a.mix_b)[h]))
                                : to_f32<DT>(((const st *)a.fixed_mix)[h]);
            s_gate[1] = rnd_st<DT>(1.f / (1.f + expf(-ml)));
        }
    }
    float qr = 0.f, kr = 0.f;
    if (a.rope && tid < R) {
        constexpr int half = R / 2;
        const int pd = tid < half ? tid + half : tid - half;
        const int64_t prow = (int64_t)min(pos, a.rope_rows - 1) * R;
        const float c = load_any(a.rcos, a.rope_dt, prow + tid), sn = load_any(a.rsin, a.rope_dt, prow + tid);
        qr = rope1<DT>(s_q[tid], s_q[pd], tid < half, c, sn, a.rope_dt);
        kr = rope1<DT>(s_k[tid], s_k[pd], tid < half, c, sn, a.rope_dt);
    }
    __syncthreads();  // the gates and partners above read the unrotated values
    if (a.rope && tid < R) {
        s_q[tid] = qr;
        s_k[tid] = kr;
    }
    __syncthreads();
    // cache append at row pos (read by later calls only: this call streams rows [0, pos))
    st *ck = (st *)a.cache_k + b * a.ck_sb + h * a.ck_sh + (int64_t)pos * a.ck_sl;
    st *cv = (st *)a.cache_v + b * a.cv_sb + h * a.cv_sh + (int64_t)pos * a.cv_sl;
    for (int i = tid; i < R; i += kThreads) ck[i] = from_f32<DT>(s_k[i]);
    for (int i = tid; i < D; i += kThreads) cv[i] = from_f32<DT>(s_v[i]);
    // the new token's partial
    float *pacc = a.ws_acc + ((int64_t)bh * a.nslot + a.n_split) * D;
    for (int i = tid; i < D; i += kThreads) pacc[i] = s_v[i];
    if (tid < 64) {
        const float dot = wave_sum(lane < R ? s_q[lane] * s_k[lane] : 0.f);
        if (lane == 0) *(float2 *)(a.ws_ml + ((int64_t)bh * a.nslot + a.n_split) * 2) = make_float2(dot * a.qscale, 1.f);
    }
    // GLA update on the inlier channels (not rotated) with the token's decay
    const float lg = s_gate[0];
    for (int i = tid; i < J; i += kThreads) {
        float e = lg;
        if (a.log_alpha) e = lg * expf(load_any(a.log_alpha, a.la_dt, h * a.la_sh + i * a.la_sj));
        s_g[i] = expf(e);
    }
    __syncthreads();
    float *sout = a.state_out + b * a.so_sb + h * a.so_sh;
    const f32x4 vv = {s_v[d4], s_v[d4 + 1], s_v[d4 + 2], s_v[d4 + 3]};
    f32x4 yp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
        const int j = jr + i * RG;
        if (j < J) {
            const f32x4 sn = s_g[j] * srow[i] + s_k[R + j] * vv;
            *(f32x4 *)(sout + j * D + d4) = sn;
            yp += s_q[R + j] * sn;
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) s_red[jr * D + d4 + c] = yp[c];
    __syncthreads();
    float y = 0.f;
    if (tid < D) {
#pragma unroll
        for (int r = 0; r < RG; ++r) y += s_red[r * D + tid];
    }
    float ss = wave_sum(y * y);  // D <= 128: waves 0 and 1 hold y
    __shared__ float s_ss[kWaves];
    if (lane == 0) s_ss[tid >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) ss += s_ss[w];
    const float mix = s_gate[1];
    float *z = a.ws_z + bh * (D + 4);
    if (tid < D) {
        const float nw = load_any(a.norm_w, a.nw_dt, h * a.nw_sh + tid * a.nw_sd);
        z[tid] = (1.f - mix) * (y * rsqrtf(ss / (float)D + a.eps) * nw);
    }
    if (tid == 0) z[D] = mix;
}

template <int DT, int D, int R, bool PRO>
__global__ __launch_bounds__(kThreads) void decode_stream_kernel(DecodeKArgs a) {
    using st = typename Stor<DT>::type;
    using G = Geometry<DT, D>;
    constexpr int EPV = G::EPV, LPR = G::LPR, TT = G::TT;
    constexpr int KL = R / EPV;          // lanes per K row
    constexpr int NKL = TT * KL / 64;    // K vectors per lane per tile
    constexpr int NVL = 8;               // V vectors per lane per tile
    static_assert(KL >= 1 && KL <= LPR && (64 % KL) == 0 && NKL >= 1, "unsupported (D, R) geometry");
    __shared__ float s_acc[kWaves][D];
    __shared__ float s_ml[kWaves][2];

    const int nbh = a.B * a.H;
    if ((int)blockIdx.x < nbh) {
        if constexpr (PRO) state_block_pro<DT, D, R>(a, blockIdx.x);
        else state_block<DT, D, R>(a, blockIdx.x);
        return;
    }
    const int bh = (blockIdx.x - nbh) / a.n_split, split = (blockIdx.x - nbh) % a.n_split;
    const int b = bh / a.H, h = bh % a.H;
    const int seq_len = current_len(a);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pk = lane % KL, pv = lane % LPR;
    const int tpw = a.tps / kWaves;
    const int ws = split * a.tps + wave * tpw;
    // with the prologue the newest row is the state block's partial
    const int we = min(ws + tpw, PRO ? max(seq_len - 1, 0) : seq_len);

    const st *ckh = (const st *)a.cache_k + b * a.ck_sb + h * a.ck_sh;
    const st *cvh = (const st *)a.cache_v + b * a.cv_sb + h * a.cv_sh;
    const int krow = (int)(a.ck_sl * sizeof(st)), vrow = (int)(a.cv_sl * sizeof(st));
    const int nvalid = we > 0 ? we : 0;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void *)ckh, 0, nvalid * krow, kBufFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void *)cvh, 0, nvalid * vrow, kBufFlags);
    const int koff0 = (lane / KL) * krow + pk * 16;
    const int voff0 = (lane / LPR) * vrow + pv * 16;

    u32x4 kb[NKL], vb[NVL];
    auto load_tile = [&](int t0, u32x4 *kd, u32x4 *vd) {
#pragma unroll
        for (int i = 0; i < NKL; ++i)
            kd[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rk, koff0 + (t0 + 64 * i / KL) * krow, 0, kLoadNT));
#pragma unroll
        for (int i = 0; i < NVL; ++i)
            vd[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rv, voff0 + (t0 + i * (64 / LPR)) * vrow, 0, kLoadNT));
    };
    // The first tile's cache rows are requested before q: they do not depend on
    // it, and q (with the rotary rows of the prologue variant) then arrives
    // within the same memory round trip.
    if (ws < we) load_tile(ws, kb, vb);

    // raw q elements, converted only after the rotary rows are requested, so
    // no wait for them sits between the loads
    const st *qp = (const st *)a.q + b * a.q_sb + h * a.q_sh;
    st qraw[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) qraw[e] = qp[(pk * EPV + e) * a.q_sd];
    // the prologue variant's rotary elements of this lane (one dtype test for all)
    float cs[EPV], sn[EPV];
    if constexpr (PRO) {
        if (a.rope) {
            const int64_t prow = (int64_t)min(max(seq_len - 1, 0), a.rope_rows - 1) * R + pk * EPV;
            if (a.rope_dt == HOFA_F32) {
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    cs[e] = ((const float *)a.rcos)[prow + e];
                    sn[e] = ((const float *)a.rsin)[prow + e];
                }
            } else {
                uint16_t cr[EPV], sr[EPV];
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    cr[e] = ((const uint16_t *)a.rcos)[prow + e];
                    sr[e] = ((const uint16_t *)a.rsin)[prow + e];
                }
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    cs[e] = a.rope_dt == HOFA_BF16 ? bf16_bits_to_f32(cr[e]) : to_f32<HOFA_F16>(cr[e]);
                    sn[e] = a.rope_dt == HOFA_BF16 ? bf16_bits_to_f32(sr[e]) : to_f32<HOFA_F16>(sr[e]);
                }
            }
        }
    }

    float qv[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) qv[e] = to_f32<DT>(qraw[e]);
    if constexpr (PRO) {  // rotate this lane's q elements; the partner half sits KL/2 lanes away
        static_assert(KL >= 2, "RoPE partner lanes");
        if (a.rope) {
            float pq[EPV];
#pragma unroll
            for (int e = 0; e < EPV; ++e) pq[e] = __shfl_xor(qv[e], KL / 2);
#pragma unroll
            for (int e = 0; e < EPV; ++e) qv[e] = rope1<DT>(qv[e], pq[e], pk < KL / 2, cs[e], sn[e], a.rope_dt);
        }
    }
#pragma unroll
    for (int e = 0; e < EPV; ++e) qv[e] *= a.qscale;

    float m_run = -INFINITY, l_run = 0.f;
    float acc[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[e] = 0.f;
    for (int t0 = ws; t0 < we; t0 += TT) {
        u32x4 kn[NKL], vn[NVL];
        const bool more = t0 + TT < we;
        if (more) load_tile(t0 + TT, kn, vn);

        float s[NKL];
#pragma unroll
        for (int i = 0; i < NKL; ++i) {
            float kf[EPV];
            unpack16<DT>(kb[i], kf);
            float acc_s = 0.f;
#pragma unroll
            for (int e = 0; e < EPV; ++e) acc_s = fmaf(qv[e], kf[e], acc_s);
#pragma unroll
            for (int off = 1; off < KL; off <<= 1) acc_s += __shfl_xor(acc_s, off);
            const int tok = t0 + (lane + 64 * i) / KL;
            s[i] = tok < we ? acc_s : -INFINITY;
        }
        // The reference m_run moves (with a wave max and a rescale) only when a
        // score exceeds it by more than kRefTau; otherwise P <= 2^kRefTau.
        float mt = s[0];
#pragma unroll
        for (int i = 1; i < NKL; ++i) mt = fmaxf(mt, s[i]);
        if (__ballot(mt > m_run + kRefTau)) {  // wave-uniform; always taken on the first tile
            const float mn = fmaxf(m_run, wave_max(mt));
            const float sc = fast_exp2(m_run - mn);  // 0 while acc and l are still empty
#pragma unroll
            for (int e = 0; e < EPV; ++e) acc[e] *= sc;
            l_run *= sc;
            m_run = mn;
        }
        float p[NKL];
#pragma unroll
        for (int i = 0; i < NKL; ++i) p[i] = fast_exp2(s[i] - m_run);
        float lsum = 0.f;
#pragma unroll
        for (int i = 0; i < NVL; ++i) {
            // the score of V-token i lives in register (i*KL)/LPR of the lane heading its K row
            const int src = ((lane / LPR + i * (64 / LPR)) * KL) & 63;
            const float pi = __shfl(p[(i * KL) / LPR], src);
            float vf[EPV];
            unpack16<DT>(vb[i], vf);
#pragma unroll
            for (int e = 0; e < EPV; ++e) acc[e] = fmaf(pi, vf[e], acc[e]);
            lsum += pi;
        }
        l_run += lsum;
        if (more) {
#pragma unroll
            for (int i = 0; i < NKL; ++i) kb[i] = kn[i];
#pragma unroll
            for (int i = 0; i < NVL; ++i) vb[i] = vn[i];
        }
    }
    // Lanes sharing pv hold disjoint token subsets of the same dims.
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[e] += __shfl_xor(acc[e], off);
        l_run += __shfl_xor(l_run, off);
    }
    if (lane < LPR) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) s_acc[wave][lane * EPV + e] = acc[e];
    }
    if (lane == 0) {
        s_ml[wave][0] = m_run;
        s_ml[wave][1] = l_run;
    }
    __syncthreads();
    // Merge the four waves; one partial per block.
    float M = s_ml[0][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_ml[w][0]);
    float wgt[kWaves], L = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        wgt[w] = s_ml[w][0] == -INFINITY ? 0.f : fast_exp2(s_ml[w][0] - M);
        L += wgt[w] * s_ml[w][1];
    }
    float *pacc = a.ws_acc + ((int64_t)bh * a.nslot + split) * D;
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) o += wgt[w] * s_acc[w][d];
        pacc[d] = o;
    }
    if (threadIdx.x == 0) *(float2 *)(a.ws_ml + ((int64_t)bh * a.nslot + split) * 2) = make_float2(M, L);
}

// One wave per head.  Every global load is issued before any of them is
// consumed: lane p holds partial p's (max, denominator); the numerators of all
// NS partials for the lane's dims sit in registers (indices past n_split are
// clamped and weigh zero).
template <int DT, int D, int NS>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeKArgs a) {
    using st = typename Stor<DT>::type;
    constexpr int DPL = D / 64;  // dims per lane
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int lane = threadIdx.x;
    const int ns = a.nslot;
    const float *pacc = a.ws_acc + (int64_t)bh * ns * D;
    const float2 ml = lane < ns ? ((const float2 *)a.ws_ml)[(int64_t)bh * ns + lane] : make_float2(-INFINITY, 0.f);
    float av[NS][DPL];
#pragma unroll
    for (int p = 0; p < NS; ++p) {
        const int pc = min(p, ns - 1);
#pragma unroll
        for (int c = 0; c < DPL; ++c) av[p][c] = pacc[pc * D + lane + 64 * c];
    }
    const float *zp = a.ws_z + bh * (D + 4);
    float z[DPL];
#pragma unroll
    for (int c = 0; c < DPL; ++c) z[c] = zp[lane + 64 * c];
    const float mix = zp[D];

    const float M = wave_max(ml.x);
    const float w = ml.x == -INFINITY ? 0.f : fast_exp2(ml.x - M);
    const float L = wave_sum(w * ml.y);
    float ao[DPL];
#pragma unroll
    for (int c = 0; c < DPL; ++c) ao[c] = 0.f;
#pragma unroll
    for (int p = 0; p < NS; ++p) {
        const float wp = p < ns ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), p)) : 0.f;
#pragma unroll
        for (int c = 0; c < DPL; ++c) ao[c] = fmaf(wp, av[p][c], ao[c]);
    }
    const float inv_l = 1.f / (L > 0.f ? L : 1.f);
#pragma unroll
    for (int c = 0; c < DPL; ++c)
        ((st *)a.y)[b * a.y_sb + h * a.y_sh + (lane + 64 * c) * a.y_sd] = from_f32<DT>(fmaf(mix, ao[c] * inv_l, z[c]));
}

// ------------------------------------------------------------------ host
int elem_size(int dt) { return dt == HOFA_F32 ? 4 : 2; }

int tile_tokens(int dt, int D) { return 64 * 8 / (D * elem_size(dt) / 16); }

int validate(const hofa_decode_args_t *a) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_decode: args is NULL");
    HOFA_REQUIRE(a->B > 0 && a->H > 0, HOFA_EINVAL, "hofa_decode: B=%d H=%d must be positive", a->B, a->H);
    HOFA_REQUIRE(a->D == 64 || a->D == 128, HOFA_EUNSUPPORTED, "hofa_decode: head dim D=%d not in {64,128}", a->D);
    HOFA_REQUIRE((a->R == 16 || a->R == 32 || a->R == 64) && a->R < a->D && 8 * a->R >= a->D, HOFA_EUNSUPPORTED,
                 "hofa_decode: outlier dims R=%d unsupported for D=%d (need R in {16,32,64}, R<D, 8R>=D)", a->R, a->D);
    const int dt = a->q.dtype;
    HOFA_REQUIRE(dt == HOFA_F32 || dt == HOFA_BF16 || dt == HOFA_F16, HOFA_EINVAL, "hofa_decode: bad dtype %d", dt);
    HOFA_REQUIRE(a->k.dtype == dt && a->v.dtype == dt && a->cache_k.dtype == dt && a->cache_v.dtype == dt &&
                     a->y.dtype == dt,
                 HOFA_EINVAL, "hofa_decode: q, k, v, caches and y must share one dtype");
    HOFA_REQUIRE(a->state_in.dtype == HOFA_F32 && a->state_out.dtype == HOFA_F32, HOFA_EINVAL,
                 "hofa_decode: states must be float32");
    HOFA_REQUIRE(a->q.data && a->k.data && a->v.data && a->cache_k.data && a->cache_v.data && a->state_in.data &&
                     a->state_out.data && a->log_gamma.data && a->mix.data && a->norm_w.data && a->y.data,
                 HOFA_EINVAL, "hofa_decode: NULL tensor pointer");
    HOFA_REQUIRE(a->state_in.data != a->state_out.data, HOFA_EINVAL, "hofa_decode: state_out must not alias state_in");
    const int J = a->D - a->R;
    HOFA_REQUIRE(a->state_in.stride[3] == 1 && a->state_in.stride[2] == a->D && a->state_out.stride[3] == 1 &&
                     a->state_out.stride[2] == a->D,
                 HOFA_EINVAL, "hofa_decode: states must be contiguous [B,H,%d,%d]", J, a->D);
    HOFA_REQUIRE(((uintptr_t)a->state_in.data % 16) == 0 && ((uintptr_t)a->state_out.data % 16) == 0 &&
                     (a->state_in.stride[1] % 4) == 0 && (a->state_in.stride[0] % 4) == 0 &&
                     (a->state_out.stride[1] % 4) == 0 && (a->state_out.stride[0] % 4) == 0,
                 HOFA_EINVAL, "hofa_decode: states must be 16-byte aligned");
    const int es = elem_size(dt);
    HOFA_REQUIRE(a->cache_k.stride[3] == 1 && a->cache_v.stride[3] == 1, HOFA_EINVAL,
                 "hofa_decode: caches must be contiguous in the last dim");
    for (const hofa_view_t *c : {&a->cache_k, &a->cache_v}) {
        HOFA_REQUIRE(((uintptr_t)c->data % 16) == 0 && (c->stride[0] * es) % 16 == 0 && (c->stride[1] * es) % 16 == 0 &&
                         (c->stride[2] * es) % 16 == 0,
                     HOFA_EINVAL, "hofa_decode: cache rows must be 16-byte aligned");
    }
    const int L = a->seq_len_dev ? a->cache_len : a->seq_len;
    HOFA_REQUIRE(L >= 1, HOFA_EINVAL, "hofa_decode: seq_len=%d cache_len=%d must be >= 1", a->seq_len, a->cache_len);
    HOFA_REQUIRE(a->seq_len_dev || a->cache_len <= 0 || a->seq_len <= a->cache_len, HOFA_EINVAL,
                 "hofa_decode: seq_len=%d exceeds cache_len=%d", a->seq_len, a->cache_len);
    HOFA_REQUIRE((int64_t)L * a->cache_v.stride[2] * es < (int64_t)1 << 31 &&
                     (int64_t)L * a->cache_k.stride[2] * es < (int64_t)1 << 31,
                 HOFA_EUNSUPPORTED, "hofa_decode: one head's cache must span less than 2 GiB");
    HOFA_REQUIRE(a->split_k >= 0 && a->split_k <= kMaxSplit, HOFA_EINVAL, "hofa_decode: split_k=%d not in [0,%d]",
                 a->split_k, kMaxSplit);
    return HOFA_OK;
}

// Splits per head (each wave at least two tiles).
void plan(const hofa_decode_args_t *a, int *n_split, int *tps) {
    const int unit = kWaves * tile_tokens(a->q.dtype, a->D);
    const int L = a->seq_len_dev ? a->cache_len : a->seq_len;
    int n;
    if (a->split_k > 0) {
        n = a->split_k;
    } else {
        // About twelve stream blocks per CU: small blocks balance the CUs and
        // keep many loads in flight (measured at cfg3: B=4 streams 4% faster
        // than at two blocks per CU); at most 48 partials per head keep the
        // merge short.
        const int bh = a->B * a->H;
        const int target = (12 * device_cu_count() + bh - 1) / bh;
        const int max_by_len = std::max(1, L / (2 * unit));
        n = std::max(1, std::min(std::min(target, max_by_len), kPlanMaxSplit));
    }
    int t = (L + n - 1) / n;
    t = (t + unit - 1) / unit * unit;
    *tps = t;
    *n_split = (L + t - 1) / t;
}

size_t acc_bytes(const hofa_decode_args_t *a, int n_split) { return (size_t)a->B * a->H * n_split * a->D * 4; }

size_t ml_bytes(const hofa_decode_args_t *a, int n_split) { return (size_t)a->B * a->H * n_split * 2 * 4; }

size_t ws_bytes(const hofa_decode_args_t *a, int n_split) {
    return acc_bytes(a, n_split) + ml_bytes(a, n_split) + (size_t)a->B * a->H * (a->D + 4) * 4;
}

template <int DT, int D, int R, bool PRO>
void launch(const DecodeKArgs &k, hipStream_t s) {
    const int bh = k.B * k.H;
    hipLaunchKernelGGL((decode_stream_kernel<DT, D, R, PRO>), dim3(bh + bh * k.n_split), dim3(kThreads), 0, s, k);
    if (k.nslot <= 8) hipLaunchKernelGGL((decode_merge_kernel<DT, D, 8>), dim3(bh), dim3(64), 0, s, k);
    else if (k.nslot <= 16) hipLaunchKernelGGL((decode_merge_kernel<DT, D, 16>), dim3(bh), dim3(64), 0, s, k);
    else if (k.nslot <= 32) hipLaunchKernelGGL((decode_merge_kernel<DT, D, 32>), dim3(bh), dim3(64), 0, s, k);
    else hipLaunchKernelGGL((decode_merge_kernel<DT, D, 64>), dim3(bh), dim3(64), 0, s, k);
}

template <int DT, bool PRO>
int dispatch(const DecodeKArgs &k, int D, int R, hipStream_t s) {
    if (D == 64 && R == 16) launch<DT, 64, 16, PRO>(k, s);
    else if (D == 64 && R == 32) launch<DT, 64, 32, PRO>(k, s);
    else if (D == 128 && R == 16) launch<DT, 128, 16, PRO>(k, s);
    else if (D == 128 && R == 32) launch<DT, 128, 32, PRO>(k, s);
    else if (D == 128 && R == 64) launch<DT, 128, 64, PRO>(k, s);
    else return HOFA_EUNSUPPORTED;
    return HOFA_OK;
}

}  // namespace
}  // namespace hofa

using namespace hofa;

extern "C" int hofa_decode_plan(const hofa_decode_args_t *a, int32_t *split_k, int32_t *tokens_per_split) {
    int rc = validate(a);
    if (rc) return rc;
    int n, t;
    plan(a, &n, &t);
    if (split_k) *split_k = n;
    if (tokens_per_split) *tokens_per_split = t;
    return HOFA_OK;
}

extern "C" size_t hofa_decode_workspace_bytes(const hofa_decode_args_t *a) {
    if (validate(a)) return 0;
    int n, t;
    plan(a, &n, &t);
    return ws_bytes(a, n);
}

extern "C" size_t hofa_decode_fused_workspace_bytes(const hofa_decode_args_t *a) {
    if (validate(a)) return 0;
    int n, t;
    plan(a, &n, &t);
    return ws_bytes(a, n + 1);  // plus the new token's partial per head
}

namespace {

int run_decode(const hofa_decode_args_t *a, const hofa_decode_prologue_args_t *p, void *workspace,
               size_t workspace_bytes, void *stream) {
    int rc = validate(a);
    if (rc) return rc;
    int n, t;
    plan(a, &n, &t);
    const int nslot = p ? n + 1 : n;
    HOFA_REQUIRE(nslot <= kMaxSplit, HOFA_EINVAL, "hofa_decode_fused: %d splits plus the new token exceed %d", n,
                 kMaxSplit);
    const size_t need = ws_bytes(a, nslot);
    HOFA_REQUIRE(workspace && workspace_bytes >= need, HOFA_EWORKSPACE,
                 "hofa_decode: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
    HOFA_REQUIRE(((uintptr_t)workspace % 16) == 0, HOFA_EWORKSPACE, "hofa_decode: workspace must be 16-byte aligned");

    DecodeKArgs k{};
    k.q = a->q.data; k.k = a->k.data; k.v = a->v.data;
    k.cache_k = a->cache_k.data; k.cache_v = a->cache_v.data;
    k.state_in = (const float *)a->state_in.data;
    k.state_out = (float *)a->state_out.data;
    k.log_gamma = a->log_gamma.data; k.mix = a->mix.data; k.norm_w = a->norm_w.data;
    k.log_alpha = a->log_alpha.data;
    k.y = (void *)a->y.data;
    k.seq_len_dev = a->seq_len_dev;
    k.ws_acc = (float *)workspace;
    k.ws_ml = (float *)((char *)workspace + acc_bytes(a, nslot));
    k.ws_z = (float *)((char *)workspace + acc_bytes(a, nslot) + ml_bytes(a, nslot));
    k.q_sb = a->q.stride[0]; k.q_sh = a->q.stride[1]; k.q_sd = a->q.stride[3];
    k.k_sb = a->k.stride[0]; k.k_sh = a->k.stride[1]; k.k_sd = a->k.stride[3];
    k.v_sb = a->v.stride[0]; k.v_sh = a->v.stride[1]; k.v_sd = a->v.stride[3];
    k.ck_sb = a->cache_k.stride[0]; k.ck_sh = a->cache_k.stride[1]; k.ck_sl = a->cache_k.stride[2];
    k.cv_sb = a->cache_v.stride[0]; k.cv_sh = a->cache_v.stride[1]; k.cv_sl = a->cache_v.stride[2];
    k.st_sb = a->state_in.stride[0]; k.st_sh = a->state_in.stride[1];
    k.so_sb = a->state_out.stride[0]; k.so_sh = a->state_out.stride[1];
    k.lg_sb = a->log_gamma.stride[0]; k.lg_sh = a->log_gamma.stride[1]; k.lg_dt = a->log_gamma.dtype;
    k.mg_sb = a->mix.stride[0]; k.mg_sh = a->mix.stride[1]; k.mg_dt = a->mix.dtype;
    k.nw_sh = a->norm_w.stride[0]; k.nw_sd = a->norm_w.stride[1]; k.nw_dt = a->norm_w.dtype;
    k.la_sh = a->log_alpha.stride[0]; k.la_sj = a->log_alpha.stride[1]; k.la_dt = a->log_alpha.dtype;
    k.y_sb = a->y.stride[0]; k.y_sh = a->y.stride[1]; k.y_sd = a->y.stride[3];
    k.B = a->B; k.H = a->H;
    k.seq_len = a->seq_len; k.cache_len = a->seq_len_dev ? a->cache_len : a->seq_len;
    k.n_split = n; k.tps = t; k.nslot = nslot;
    if (p) {
        k.gate_w = p->gate_w; k.gate_b = p->gate_b; k.mix_w = p->mix_w; k.mix_b = p->mix_b;
        k.fixed_mix = p->fixed_mix; k.rcos = p->cos; k.rsin = p->sin;
        k.rope = p->cos != nullptr; k.rope_dt = p->rope_dtype; k.rope_rows = p->rope_rows;
    }
    k.qscale = a->sm_scale * kLog2e;
    k.eps = a->eps;

    hipStream_t s = (hipStream_t)stream;
    if (p) {
        rc = a->q.dtype == HOFA_BF16 ? dispatch<HOFA_BF16, true>(k, a->D, a->R, s)
                                     : dispatch<HOFA_F16, true>(k, a->D, a->R, s);
    } else {
        switch (a->q.dtype) {
            case HOFA_F32: rc = dispatch<HOFA_F32, false>(k, a->D, a->R, s); break;
            case HOFA_BF16: rc = dispatch<HOFA_BF16, false>(k, a->D, a->R, s); break;
            default: rc = dispatch<HOFA_F16, false>(k, a->D, a->R, s); break;
        }
    }
    if (rc) {
        set_error("hofa_decode: no kernel for this (D, R)");
        return rc;
    }
    return check_launch("hofa_decode");
}

}  // namespace

extern "C" int hofa_decode(const hofa_decode_args_t *a, void *workspace, size_t workspace_bytes, void *stream) {
    return run_decode(a, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int hofa_decode_fused(const hofa_decode_args_t *a, const hofa_decode_prologue_args_t *p, void *workspace,
                                 size_t workspace_bytes, void *stream) {
    HOFA_REQUIRE(a && p, HOFA_EINVAL, "hofa_decode_fused: args is NULL");
    HOFA_REQUIRE(p->B == a->B && p->H == a->H && p->D == a->D && p->R == a->R && p->dtype == a->q.dtype, HOFA_EINVAL,
                 "hofa_decode_fused: prologue (B, H, D, R, dtype) must match the decode arguments");
    HOFA_REQUIRE(a->q.dtype == HOFA_BF16 || a->q.dtype == HOFA_F16, HOFA_EUNSUPPORTED,
                 "hofa_decode_fused: dtype %d must be bf16 or f16", a->q.dtype);
    HOFA_REQUIRE(p->gate_w && p->gate_b && ((p->mix_w && p->mix_b) || p->fixed_mix), HOFA_EINVAL,
                 "hofa_decode_fused: need gate_w, gate_b and mix_w + mix_b or fixed_mix");
    HOFA_REQUIRE(!p->cos == !p->sin && (!p->cos || (p->rope_rows > 0 && (p->rope_dtype == HOFA_F32 ||
                                                                         p->rope_dtype == p->dtype))),
                 HOFA_EINVAL, "hofa_decode_fused: RoPE tables need cos and sin, rope_rows > 0, f32 or the dtype");
    return run_decode(a, p, workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------------ allocation-free entry point
// hofa_decode_static: the split-K partials live in `scratch`, one file-scope
// device array per GPU, instead of a caller workspace.  Host code never
// passes the array's name to a kernel (on the host it is a stand-in, not a
// device address); the address comes from hipGetSymbolAddress, called once
// per device with that device current, and is kept per device.
static __device__ __align__(256) unsigned char scratch[HOFA_DECODE_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of this GPU's `scratch` (resolved on first use).
int scratch_for_stream(hipStream_t stream, void **out) {
    int dev = -1;
    if (stream) {
        HOFA_REQUIRE(hipStreamGetDevice(stream, &dev) == hipSuccess, HOFA_ELAUNCH,
                     "hofa_decode_static: hipStreamGetDevice failed");
    } else {
        HOFA_REQUIRE(hipGetDevice(&dev) == hipSuccess, HOFA_ELAUNCH, "hofa_decode_static: hipGetDevice failed");
    }
    HOFA_REQUIRE(dev >= 0 && dev < kMaxDevices, HOFA_EUNSUPPORTED, "hofa_decode_static: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        HOFA_REQUIRE(hipGetDevice(&cur) == hipSuccess, HOFA_ELAUNCH, "hofa_decode_static: hipGetDevice failed");
        if (cur != dev)
            HOFA_REQUIRE(hipSetDevice(dev) == hipSuccess, HOFA_ELAUNCH, "hofa_decode_static: hipSetDevice(%d) failed",
                         dev);
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        HOFA_REQUIRE(e == hipSuccess && ptr, HOFA_ELAUNCH, "hofa_decode_static: hipGetSymbolAddress failed: %s",
                     hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return HOFA_OK;
}

}  // namespace

extern "C" int hofa_decode_static(const hofa_decode_args_t *a, void *stream) {
    int rc = validate(a);
    if (rc) return rc;
    int n, t;
    plan(a, &n, &t);
    const size_t need = ws_bytes(a, n);
    HOFA_REQUIRE(need <= (size_t)HOFA_DECODE_STATIC_SCRATCH_BYTES, HOFA_EWORKSPACE,
                 "hofa_decode_static: this call needs %zu bytes of scratch, more than the %zu-byte static "
                 "array (B*H=%d heads, %d splits); use hofa_decode with a workspace",
                 need, (size_t)HOFA_DECODE_STATIC_SCRATCH_BYTES, a->B * a->H, n);
    void *ptr = nullptr;
    rc = scratch_for_stream((hipStream_t)stream, &ptr);
    if (rc) return rc;
    return run_decode(a, nullptr, ptr, (size_t)HOFA_DECODE_STATIC_SCRATCH_BYTES, stream);
}

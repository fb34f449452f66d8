// Inlier-pathway prefill for gfx950: chunked gated linear attention (GLA)
// over channels [R, D) of Q/K with full-width V, 64-token chunks.
//
// Replaces chunk_gla_inlier_fwd / chunk_gla_fwd_kernel (src/chunk_gla_inlier.py:6-237),
// which walks all chunks of one head serially in one program.  Here the
// chunks of every head run in parallel and only an element-wise fp32 scan is
// sequential over chunks:
//
//   1. gla_state_kernel   grid (B*H*nc), 4 waves: per chunk, in-chunk
//      inclusive cumsum G of the log decay (fp32, see Decay), then
//        dS^T[D x J] = V_c^T (K_c (.) exp(G_last - G))        v_mfma_f32_16x16x32
//      every exponent <= 0.  Writes dS^T and G_last.
//   2. gla_scan_kernel    grid (B*H, D/16): S_in(c) = S, S <- exp(G_last) S + dS,
//      writes S_in(c) transposed as a hi/lo pair of 16-bit operands (one bf16
//      plane with round_operands; for a backward pass also untransposed as a
//      second pair) and the final fp32 state.
//   3. gla_out_kernel     grid (B*H*nc), 2 waves x 32 query rows:
//        A^T[key, query] = K~ Q~^T     K~ = K (.) exp(-G), Q~ = Q (.) exp(G)   (masked key <= query)
//        Y^T[dv, query]  = V_c^T A^T + S_in^T Q~^T                           v_mfma_f32_32x32x16
//      each lane owns one query row, so the fused epilogue
//      (1 - mix) * gla_scale * RMSNorm(Y) (src/chunk_gla_inlier.py:130-141)
//      reduces over D inside a lane pair.  K~ grows like exp(-G); chunks
//      whose decay range exceeds kSafeRange form A^T element-wise from
//      differences G_q - G_k <= 0 in the same launch (a block-uniform branch).
// By default every matrix-core product takes its operands as hi + lo pairs
// of bf16 values (x ~ hi + lo, see split8), i.e. about 16 mantissa bits in
// the f32 exponent range: the result tracks an fp32 computation (f16 inputs
// use the same bf16 pairs).  With round_operands (16-bit inputs, no backward
// pass) each operand and the entering state are rounded to bf16 once, as the
// reference's kernel rounds them, and the state is stored as one bf16 plane.
#include "hofa_gla_common.h"

namespace hofa {
namespace {

using namespace gla;
constexpr int NT = 128;  // threads of the output kernel

// One block per (head, 16 value rows): thread (dv, j4) carries S[j4..j4+3][dv]
// in registers across the chunks, with the loads of the next kScanPF chunks
// in flight.  Plane 0 (and 1) of S^T (j contiguous) are stored directly;
// planes 2/3 (S, d contiguous), written only for a backward pass, go through
// a double-buffered LDS transpose so that both layouts leave with contiguous
// stores.
constexpr int kScanPF = 8;

// NPW: the planes written per chunk (planes_written of a.nplanes), fixed at
// compile time so the chunk loop has no branch: a branch around the stores
// leaves the compiler's memory-counter waits conservative, and the loads of
// the next chunks would be waited for at every chunk.
template <int DT, int D, int J, int NPW>
__global__ __launch_bounds__(kScanRows * J / 4) void gla_scan_kernel(GlaK a) {
    __shared__ __attribute__((aligned(16))) uint16_t sT[2][2][J * kScanPitch];
    const int bh = blockIdx.x, tid = threadIdx.x;
    const int dvl = tid / (J / 4), j4 = (tid % (J / 4)) * 4;
    const int dv0 = blockIdx.y * kScanRows, dv = dv0 + dvl;
    const int nc = a.nc;
    f32x4 S = {0.f, 0.f, 0.f, 0.f};
    const int64_t base = (int64_t)bh * nc;
    f32x4 ds[kScanPF], gl[kScanPF];  // a rolling window: slot u holds chunk c = u (mod kScanPF)
    auto fetch = [&](int u, int c) {
        c = min(c, nc - 1);  // past the end: a harmless reload of the last chunk
        ds[u] = *(const f32x4 *)(a.ws_ds + (base + c) * D * J + dv * J + j4);
        gl[u] = *(const f32x4 *)(a.ws_gl + (base + c) * J + j4);
    };
#pragma unroll
    for (int u = 0; u < kScanPF; ++u) fetch(u, u);
    for (int c0 = 0; c0 < nc; c0 += kScanPF) {
#pragma unroll
        for (int u = 0; u < kScanPF; ++u) {
            const int c = c0 + u;
            if (c >= nc) break;  // block-uniform
            const f32x4 d = ds[u], g = gl[u];
            fetch(u, c + kScanPF);
            store_state_tile<DT, D, J>(a.s_in + (base + c) * a.nplanes * D * J, NPW, dv0,
                                       dvl, j4, S, sT[c & 1][0], sT[c & 1][1]);
#pragma unroll
            for (int e = 0; e < 4; ++e) S[e] = fmaf(fast_exp2(g[e] * kLog2e), S[e], d[e]);
        }
    }
    const int b = bh / a.H, h = bh % a.H;
    float *so = a.state_out + b * a.so_sb + h * a.so_sh;
#pragma unroll
    for (int e = 0; e < 4; ++e) so[(j4 + e) * a.so_sj + dv * a.so_sd] = S[e];
    if (j4 < a.pad_rows)  // the zero rows of a padded state (pad_rows <= J, a multiple of 4)
#pragma unroll
        for (int e = 0; e < 4; ++e) so[(J + j4 + e) * a.so_sj + dv * a.so_sd] = 0.f;
}

// One block per chunk, 2 waves x 32 query rows.  Every global load of the
// chunk (decay, V, the wave's Q and K rows, gate inputs) is issued before the
// first barrier; the entering state is loaded while the decay is prepared.
// Chunks whose decay range exceeds kSafeRange (a block-uniform test) form
// A^T element-wise from exponent differences G_q - G_k <= 0 instead of the
// factored operands.  RND (16-bit inputs): every matrix-core operand is
// rounded to bf16 once, as the reference's Triton kernel rounds its dot
// operands (src/chunk_gla_inlier.py:96-110) and the state (S.to(dtype)), and
// the state comes as one bf16 plane; otherwise operands are hi/lo pairs.
template <int DT, int D, int J, bool GENERAL, bool RND>
__global__ __launch_bounds__(NT) void gla_out_kernel(GlaK a) {
    using in_t = typename Stor<DT>::type;
    constexpr int VP = C + 4;
    constexpr int MB = D / 32;
    constexpr int KS = J / 16;
    constexpr bool SPLIT = !RND;                   // hi/lo operand pairs
    constexpr bool VLO = kRawSplit<DT> && SPLIT;   // f32/f16 inputs also split V
    static_assert(D <= NT, "one gla_scale element per thread");
    __shared__ float sDec[Decay<J, GENERAL>::kFloats];
    __shared__ __attribute__((aligned(16))) uint16_t sVt[VLO ? 2 : 1][D * VP];
    __shared__ __attribute__((aligned(16))) float sGs[D];
    constexpr int NSP = SPLIT ? 2 : 1;
    __shared__ u32x4 sK0[NSP][KS][64];  // wave 0's K~ operand quads, read by wave 1
    const int bh = blockIdx.x / a.nc, c = blockIdx.x % a.nc;
    const int b = bh / a.H, h = bh % a.H, t0 = c * C;
    const int lane = threadIdx.x & 63, hi = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qi = 32 * w + (lane & 31);  // chunk-relative query row of this lane
    const int tq = t0 + qi;

    const in_t *qp = (const in_t *)a.q + b * a.q_sb + h * a.q_sh;
    const in_t *kp = (const in_t *)a.k + b * a.k_sb + h * a.k_sh;
    const Rows<DT> qrows(qp, a.q_st, a.T), krows(kp, a.k_st, a.T);
    const Rows<DT> vrows((const in_t *)a.v + b * a.v_sb + h * a.v_sh, a.v_st, a.T);

    // ---- issue every load of the chunk
    DecayStage<J, GENERAL, NT> dst;
    TrStage<DT, D, NT, 2> vst;
    dst.issue(a, b, h, t0);
    vst.issue(vrows, 0, t0);
    Raw8<DT> qr[KS], kr[KS];  // this lane's query row and key row (both 32 w + lane%32)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qr[ks].load(qrows, tq, a.R + 16 * ks + 8 * hi);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kr[ks].load(krows, tq, a.R + 16 * ks + 8 * hi);
    const float mixv =
        a.fuse && tq < a.T ? load_any(a.mix, a.mix_dt, b * a.m_sb + h * a.m_sh + (int64_t)tq * a.m_st) : 0.f;
    const float gsv = threadIdx.x < D && a.fuse ? load_any(a.gs, a.gs_dt, h * a.gs_sh + threadIdx.x * a.gs_sd) : 1.f;

    const Decay<J, GENERAL> dec{sDec};
    dst.commit(a, dec);
    const bool safe = dec.range() <= kSafeRange;  // block-uniform

    // K~ = K (.) exp(-G) of the wave's own key block (A operand, lane = key);
    // wave 0 also leaves it in LDS for wave 1, whose queries see both blocks
    u32x4 kq[NSP][KS];
    if (safe) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            float x[8];
            kr[ks].get(x);
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] *= fast_exp2(-dec.G(qi, 16 * ks + 8 * hi + e) * kLog2e);
            if constexpr (SPLIT) split8<OPB>(x, kq[0][ks], kq[NSP - 1][ks]);
            else kq[0][ks] = pack8<OPB>(x);
            if (w == 0)
#pragma unroll
                for (int p = 0; p < NSP; ++p) sK0[p][ks][lane] = kq[p][ks];
        }
    }

    // entering state (chunk 0 starts from zero): A operand rows dv = 32 mb + lane%32
    u32x4 sst[NSP][MB][KS];
    if (c > 0) {
        const uint16_t *sin = a.s_in + ((int64_t)bh * a.nc + c) * a.nplanes * D * J;
#pragma unroll
        for (int p = 0; p < NSP; ++p)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    sst[p][mb][ks] = *(const u32x4 *)(sin + p * D * J + (32 * mb + (lane & 31)) * J + 16 * ks + 8 * hi);
    }

    vst.template commit<VP, VLO>(sVt[0], sVt[VLO ? 1 : 0], [](int, int) { return 1.f; });
    if (threadIdx.x < D) sGs[threadIdx.x] = gsv;
    __syncthreads();

    // Q~ = Q (.) exp(G): B operand (lane = query)
    u32x4 qh[KS], ql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        float x[8];
        qr[ks].get(x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= fast_exp2(dec.G(qi, 16 * ks + 8 * hi + e) * kLog2e);
        if constexpr (SPLIT) split8<OPB>(x, qh[ks], ql[ks]);
        else qh[ks] = pack8<OPB>(x);
    }

    f32x16 y[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) y[mb][v] = 0.f;

#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {  // key blocks at or before the wave's queries
        if (kb > w) break;
        f32x16 at;
#pragma unroll
        for (int v = 0; v < 16; ++v) at[v] = 0.f;
        if (safe) {
            const bool own = kb == w;  // else wave 1 reading wave 0's block from LDS
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const u32x4 kh = own ? kq[0][ks] : sK0[0][ks][lane];
                at = mfma32<OPB>(kh, qh[ks], at);
                if constexpr (SPLIT) {
                    const u32x4 kl = own ? kq[NSP - 1][ks] : sK0[NSP - 1][ks][lane];
                    at = mfma32<OPB>(kh, ql[ks], at);
                    at = mfma32<OPB>(kl, qh[ks], at);
                }
            }
        } else {
            // element-wise: A[q, k] = sum_c q_c k_c exp(G_q,c - G_k,c), every exponent <= 0
#pragma unroll 1
            for (int ch = 0; ch < J; ++ch) {
                const float qv = tq < a.T ? to_f32<DT>(qp[(int64_t)tq * a.q_st + a.R + ch]) : 0.f;
                const float gq = dec.G(qi, ch);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int kj = 32 * kb + 8 * (v / 4) + 4 * hi + (v % 4);
                    const int tk = t0 + kj;
                    if (kj <= qi && tk < a.T) {
                        const float kv = to_f32<DT>(kp[(int64_t)tk * a.k_st + a.R + ch]);
                        at[v] = fmaf(qv * kv, fast_exp2((gq - dec.G(kj, ch)) * kLog2e), at[v]);
                    }
                }
            }
        }
        // causal mask inside the chunk (key <= query)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int kj = 32 * kb + 8 * (v / 4) + 4 * hi + (v % 4);
            if (kj > qi) at[v] = 0.f;
        }
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            u32x4 ph, pl;
            if constexpr (SPLIT) split8v<OPB>(at, 8 * k2, ph, pl);
            else ph = pack8<OPB>(at, 8 * k2);
            const int ks4 = 2 * kb + k2;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int vo = (32 * mb + (lane & 31)) * VP + ((16 * ks4 + 4 * hi) ^ tr_col_swz(32 * mb));
                const uint2 lo = *(const uint2 *)&sVt[0][vo], hi8 = *(const uint2 *)&sVt[0][vo + 8];
                const u32x4 va = {lo.x, lo.y, hi8.x, hi8.y};
                y[mb] = mfma32<OPB>(va, ph, y[mb]);
                if constexpr (SPLIT) y[mb] = mfma32<OPB>(va, pl, y[mb]);
                if constexpr (VLO) {
                    const uint2 l2 = *(const uint2 *)&sVt[VLO ? 1 : 0][vo],
                                h2 = *(const uint2 *)&sVt[VLO ? 1 : 0][vo + 8];
                    y[mb] = mfma32<OPB>(u32x4{l2.x, l2.y, h2.x, h2.y}, ph, y[mb]);
                }
            }
        }
    }
    if (c > 0) {  // inter-chunk term: S_in^T Q~^T
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                y[mb] = mfma32<OPB>(sst[0][mb][ks], qh[ks], y[mb]);
                if constexpr (SPLIT) {
                    y[mb] = mfma32<OPB>(sst[0][mb][ks], ql[ks], y[mb]);
                    y[mb] = mfma32<OPB>(sst[NSP - 1][mb][ks], qh[ks], y[mb]);
                }
            }
    }

    // ---- epilogue
    if (a.fuse) {
        float ss = 0.f;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int v = 0; v < 16; ++v) ss = fmaf(y[mb][v], y[mb][v], ss);
        ss += __shfl_xor(ss, 32);
        const float rs = rsqrtf(ss / (float)D + a.eps);
        const float f = (1.f - mixv) * rs;
        if (a.n_out && tq < a.T) {  // RMSNorm(Y_I) and 1/rms, saved for the backward pass
            in_t *nr = (in_t *)a.n_out + b * a.n_sb + h * a.n_sh + (int64_t)tq * a.n_st;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    store4<DT>(nr + 32 * mb + 8 * g + 4 * hi, y[mb][4 * g] * rs, y[mb][4 * g + 1] * rs,
                               y[mb][4 * g + 2] * rs, y[mb][4 * g + 3] * rs);
            if (hi == 0) a.rstd[(int64_t)bh * a.T + tq] = rs;
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 gs4 = *(const f32x4 *)&sGs[32 * mb + 8 * g + 4 * hi];
#pragma unroll
                for (int e = 0; e < 4; ++e) y[mb][4 * g + e] *= f * gs4[e];
            }
    }
    if (tq >= a.T) return;
    const int64_t yo = b * a.y_sb + h * a.y_sh + (int64_t)tq * a.y_st;
    if (a.y_f32) {  // unrounded result for a later single rounding (hofa_attn_fwd acc)
        float *yr = (float *)a.y + yo;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                store4<HOFA_F32>(yr + 32 * mb + 8 * g + 4 * hi, y[mb][4 * g], y[mb][4 * g + 1], y[mb][4 * g + 2],
                                 y[mb][4 * g + 3]);
    } else {
        in_t *yr = (in_t *)a.y + yo;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                store4<DT>(yr + 32 * mb + 8 * g + 4 * hi, y[mb][4 * g], y[mb][4 * g + 1], y[mb][4 * g + 2],
                           y[mb][4 * g + 3]);
    }
}

// ------------------------------------------------------------------ host
int elem_bytes(int dt) { return dt == HOFA_F32 ? 4 : 2; }

bool rows_ok(const hofa_view_t &v, int es) {
    return v.stride[3] == 1 && ((uintptr_t)v.data % 16) == 0 && (v.stride[0] * es) % 16 == 0 &&
           (v.stride[1] * es) % 16 == 0 && (v.stride[2] * es) % 16 == 0;
}

// 16-bit planes per entering state: 4 for a backward pass (chunk_states),
// one bf16 plane with rounded operands, else a hi/lo pair.
int state_planes(const hofa_gla_fwd_args_t *a) {
    if (a->chunk_states) return 4;
    return a->round_operands && a->q.dtype != HOFA_F32 ? 1 : 2;
}

struct WsLayout {
    size_t ds, gl, sin, flags, total;
};

WsLayout ws_layout(const hofa_gla_fwd_args_t *a) {
    const size_t bh = (size_t)a->B * a->H, nc = (a->T + C - 1) / C, J = a->D - a->R;
    WsLayout w{};
    w.ds = 0;
    w.gl = (bh * nc * a->D * J * 4 + 255) / 256 * 256;
    w.sin = w.gl + (bh * nc * J * 4 + 255) / 256 * 256;
    w.flags = w.sin + (a->chunk_states ? 0 : (bh * nc * state_planes(a) * a->D * J * 2 + 255) / 256 * 256);
    w.total = w.flags + (bh * nc + 255) / 256 * 256;
    return w;
}

int validate(const hofa_gla_fwd_args_t *a) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_gla_fwd: args is NULL");
    HOFA_REQUIRE(a->B > 0 && a->H > 0 && a->T > 0, HOFA_EINVAL, "hofa_gla_fwd: B=%d H=%d T=%d must be positive", a->B,
                 a->H, a->T);
    HOFA_REQUIRE(a->D == 64 || a->D == 128, HOFA_EUNSUPPORTED, "hofa_gla_fwd: head dim D=%d not in {64,128}", a->D);
    const int J = a->D - a->R;
    HOFA_REQUIRE(a->R >= 0 && J >= 16 && J % 16 == 0, HOFA_EUNSUPPORTED,
                 "hofa_gla_fwd: inlier width J=%d must be a positive multiple of 16", J);
    const int dt = a->q.dtype;
    HOFA_REQUIRE(dt == HOFA_F32 || dt == HOFA_BF16 || dt == HOFA_F16, HOFA_EINVAL, "hofa_gla_fwd: bad dtype %d", dt);
    HOFA_REQUIRE(a->k.dtype == dt && a->v.dtype == dt && (a->y.dtype == dt || a->y.dtype == HOFA_F32), HOFA_EINVAL,
                 "hofa_gla_fwd: q, k and v must share one dtype; y has it too or is float32");
    HOFA_REQUIRE(a->q.data && a->k.data && a->v.data && a->y.data && a->state_out.data, HOFA_EINVAL,
                 "hofa_gla_fwd: NULL tensor pointer");
    const int es = elem_bytes(dt);
    HOFA_REQUIRE(rows_ok(a->q, es) && rows_ok(a->k, es) && rows_ok(a->v, es) && rows_ok(a->y, elem_bytes(a->y.dtype)),
                 HOFA_EINVAL,
                 "hofa_gla_fwd: q/k/v/y need unit last stride and 16-byte aligned rows");
    HOFA_REQUIRE((a->R * es) % 16 == 0, HOFA_EINVAL, "hofa_gla_fwd: the inlier columns must start 16-byte aligned");
    HOFA_REQUIRE(a->g.data || a->log_gamma.data, HOFA_EINVAL, "hofa_gla_fwd: give log_gamma or g");
    HOFA_REQUIRE(!a->g.data || a->g.dtype == HOFA_F32, HOFA_EINVAL, "hofa_gla_fwd: g must be float32");
    HOFA_REQUIRE(!a->fuse_norm_gate || (a->mix.data && a->gla_scale.data), HOFA_EINVAL,
                 "hofa_gla_fwd: fuse_norm_gate needs mix and gla_scale");
    HOFA_REQUIRE(a->state_out.dtype == HOFA_F32, HOFA_EINVAL, "hofa_gla_fwd: state_out must be float32");
    HOFA_REQUIRE(a->state_pad_rows >= 0 && a->state_pad_rows <= a->D - a->R && a->state_pad_rows % 4 == 0, HOFA_EINVAL,
                 "hofa_gla_fwd: state_pad_rows=%d must be a multiple of 4 in [0, J]", a->state_pad_rows);
    for (const hofa_view_t *v : {&a->q, &a->k, &a->v})
        HOFA_REQUIRE((int64_t)(a->T + 2 * C) * v->stride[2] * es < (1ll << 31), HOFA_EUNSUPPORTED,
                     "hofa_gla_fwd: one head's q/k/v rows must span less than 2 GiB");
    HOFA_REQUIRE(!(a->round_operands && a->chunk_states), HOFA_EINVAL,
                 "hofa_gla_fwd: round_operands is for inference; a backward pass (chunk_states) needs hi/lo operands");
    HOFA_REQUIRE(!a->n_out.data || (a->fuse_norm_gate && a->rstd && a->n_out.dtype == dt && rows_ok(a->n_out, es)),
                 HOFA_EINVAL, "hofa_gla_fwd: n_out needs fuse_norm_gate, rstd, the dtype of y and aligned rows");
    return HOFA_OK;
}

template <int DT, int D, int J, bool GEN, bool RND>
void launch(const GlaK &k, hipStream_t s) {
    const int nblk = k.B * k.H * k.nc;
    hipLaunchKernelGGL((gla_state_kernel<DT, D, J, GEN, false, RND>), dim3(nblk), dim3(kStateThreads), 0, s, k);
    const dim3 sg(k.B * k.H, D / kScanRows), sb(kScanRows * J / 4);
    switch (planes_written<D, J>(k.nplanes)) {
        case 1: hipLaunchKernelGGL((gla_scan_kernel<DT, D, J, 1>), sg, sb, 0, s, k); break;
        case 2: hipLaunchKernelGGL((gla_scan_kernel<DT, D, J, 2>), sg, sb, 0, s, k); break;
        default: hipLaunchKernelGGL((gla_scan_kernel<DT, D, J, 4>), sg, sb, 0, s, k); break;
    }
    hipLaunchKernelGGL((gla_out_kernel<DT, D, J, GEN, RND>), dim3(nblk), dim3(NT), 0, s, k);
}

template <int DT, bool GEN, bool RND>
int dispatch(const GlaK &k, int D, int J, hipStream_t s) {
    if (D == 64 && J == 48) launch<DT, 64, 48, GEN, RND>(k, s);
    else if (D == 64 && J == 32) launch<DT, 64, 32, GEN, RND>(k, s);
    else if (D == 64 && J == 64) launch<DT, 64, 64, GEN, RND>(k, s);
    else if (D == 128 && J == 112) launch<DT, 128, 112, GEN, RND>(k, s);
    else if (D == 128 && J == 96) launch<DT, 128, 96, GEN, RND>(k, s);
    else if (D == 128 && J == 64) launch<DT, 128, 64, GEN, RND>(k, s);
    else if (D == 128 && J == 128) launch<DT, 128, 128, GEN, RND>(k, s);
    else return HOFA_EUNSUPPORTED;
    return HOFA_OK;
}

// f32 inputs always take hi/lo operand pairs.
template <int DT>
int dispatch_dt(const GlaK &k, int D, int J, bool gen, bool rnd, hipStream_t s) {
    if constexpr (DT == HOFA_F32) {
        return gen ? dispatch<DT, true, false>(k, D, J, s) : dispatch<DT, false, false>(k, D, J, s);
    } else {
        if (rnd) return gen ? dispatch<DT, true, true>(k, D, J, s) : dispatch<DT, false, true>(k, D, J, s);
        return gen ? dispatch<DT, true, false>(k, D, J, s) : dispatch<DT, false, false>(k, D, J, s);
    }
}

}  // namespace
}  // namespace hofa

using namespace hofa;

extern "C" size_t hofa_gla_fwd_workspace_bytes(const hofa_gla_fwd_args_t *a) {
    if (validate(a)) return 0;
    return ws_layout(a).total;
}

extern "C" int hofa_gla_fwd(const hofa_gla_fwd_args_t *a, void *workspace, size_t workspace_bytes, void *stream) {
    int rc = validate(a);
    if (rc) return rc;
    const WsLayout L = ws_layout(a);
    HOFA_REQUIRE(workspace && workspace_bytes >= L.total, HOFA_EWORKSPACE,
                 "hofa_gla_fwd: workspace of %zu bytes needed, got %zu", L.total, workspace_bytes);
    HOFA_REQUIRE(((uintptr_t)workspace % 256) == 0, HOFA_EWORKSPACE, "hofa_gla_fwd: workspace must be 256-byte aligned");
    HOFA_REQUIRE(!a->chunk_states || ((uintptr_t)a->chunk_states % 16) == 0, HOFA_EINVAL,
                 "hofa_gla_fwd: chunk_states must be 16-byte aligned");
    GlaK k{};
    k.q = a->q.data; k.k = a->k.data; k.v = a->v.data;
    k.lg = a->log_gamma.data; k.la = a->log_alpha.data; k.g = a->g.data;
    k.mix = a->mix.data; k.gs = a->gla_scale.data;
    k.y = (void *)a->y.data;
    k.state_out = (float *)a->state_out.data;
    char *w = (char *)workspace;
    k.ws_ds = (float *)(w + L.ds);
    k.ws_gl = (float *)(w + L.gl);
    k.s_in = a->chunk_states ? (uint16_t *)a->chunk_states : (uint16_t *)(w + L.sin);
    k.nplanes = state_planes(a);
    k.unsafe = (uint8_t *)(w + L.flags);
    k.n_out = (void *)a->n_out.data;
    k.rstd = a->n_out.data ? a->rstd : nullptr;
    k.n_sb = a->n_out.stride[0]; k.n_sh = a->n_out.stride[1]; k.n_st = a->n_out.stride[2];
    k.q_sb = a->q.stride[0]; k.q_sh = a->q.stride[1]; k.q_st = a->q.stride[2];
    k.k_sb = a->k.stride[0]; k.k_sh = a->k.stride[1]; k.k_st = a->k.stride[2];
    k.v_sb = a->v.stride[0]; k.v_sh = a->v.stride[1]; k.v_st = a->v.stride[2];
    k.y_sb = a->y.stride[0]; k.y_sh = a->y.stride[1]; k.y_st = a->y.stride[2];
    k.lg_sb = a->log_gamma.stride[0]; k.lg_sh = a->log_gamma.stride[1]; k.lg_st = a->log_gamma.stride[2];
    k.la_sh = a->log_alpha.stride[0]; k.la_sj = a->log_alpha.stride[1];
    k.g_sb = a->g.stride[0]; k.g_sh = a->g.stride[1]; k.g_st = a->g.stride[2]; k.g_sj = a->g.stride[3];
    k.m_sb = a->mix.stride[0]; k.m_sh = a->mix.stride[1]; k.m_st = a->mix.stride[2];
    k.gs_sh = a->gla_scale.stride[0]; k.gs_sd = a->gla_scale.stride[1];
    k.so_sb = a->state_out.stride[0]; k.so_sh = a->state_out.stride[1];
    k.so_sj = a->state_out.stride[2]; k.so_sd = a->state_out.stride[3];
    k.pad_rows = a->state_pad_rows;
    k.lg_dt = a->log_gamma.dtype; k.la_dt = a->log_alpha.dtype; k.mix_dt = a->mix.dtype; k.gs_dt = a->gla_scale.dtype;
    k.B = a->B; k.H = a->H; k.T = a->T; k.R = a->R;
    k.nc = (a->T + C - 1) / C;
    k.key_col0 = a->R;
    k.fuse = a->fuse_norm_gate;
    k.y_f32 = a->y.dtype == HOFA_F32 && a->q.dtype != HOFA_F32;
    k.eps = a->eps;
    const int J = a->D - a->R;
    hipStream_t s = (hipStream_t)stream;
    const bool gen = a->g.data != nullptr;
    const bool rnd = k.nplanes == 1;
    switch (a->q.dtype) {
        case HOFA_F32: rc = dispatch_dt<HOFA_F32>(k, a->D, J, gen, false, s); break;
        case HOFA_BF16: rc = dispatch_dt<HOFA_BF16>(k, a->D, J, gen, rnd, s); break;
        default: rc = dispatch_dt<HOFA_F16>(k, a->D, J, gen, rnd, s); break;
    }
    if (rc) {
        set_error("hofa_gla_fwd: no kernel for this (D, J)");
        return rc;
    }
    return check_launch("hofa_gla_fwd");
}

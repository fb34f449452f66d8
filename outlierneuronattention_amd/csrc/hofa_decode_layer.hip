// Single-token decode of a whole TransformerBlock on gfx950: the work around
// the split-K attention kernel (hofa_decode.hip), fused so that one greedy
// step of SubwordLM is about seven launches per layer instead of ~40 small
// framework kernels.
//
// Replaces, for one token (src/HybridOutlierFactorizedAttention.py):
//   TransformerBlock.forward_step (:447-451): x + attn(ln_1(x)), x + mlp(ln_2(x))
//   forward_step projections, gates, RoPE and cache append (:223-392)
//   SubwordLM lm_head (:471) and the greedy argmax / feedback of src/inference.py:220-221
//
//   rows_linear_kernel   y[b, n] = epi( LN(x)[b, :] . W[n, :] )       b < B <= 4
//       x (optionally layer-normalised, rounded to the weight dtype as
//       nn.LayerNorm's output is) is staged in LDS; each wave owns RPW output
//       rows and streams their weights with 16-byte loads, lane l taking
//       8-element pieces l, l+64, ...  The epilogue rounds like the module's
//       chain of 16-bit ops: +bias, GELU (erf), *scale on leading columns,
//       +residual, each rounded to the storage type.  With argmax every block
//       also writes its best (value, -index) key per batch row to its own slot.
//   decode_prologue_kernel   one wave per (b, h): gate and mix logits on the
//       pre-RoPE scaled Q/K (:67-95), log_gamma = logsigmoid(-gate), mix =
//       sigmoid, RoPE of the outlier channels at the device position (:365-375),
//       and the cache append at that row (:382-387); rotated q/k are written
//       back in place so the decode kernel reads them from the projection.
//   decode_advance_kernel    one block: the greedy token of every batch row
//       (the greatest of the LM head's per-block keys), its embedding row as
//       the next input, the output column, and the position counters (pos,
//       seq_len, col) advanced.
#include "hofa_mfma.h"  // pack2: two floats to one dword of 16-bit values (round to nearest even)

namespace hofa {
namespace {

constexpr int LT = 256;  // threads of the linear kernel
constexpr int LW = LT / 64;

struct RowsLinK {
    const void *x, *ln_w, *ln_b, *w, *bias, *res;
    void *y;
    unsigned long long *argmax;
    int64_t x_st, res_st, y_st;
    int B, K, N, act, scale_cols;
    float scale, ln_eps;
};

template <int DT>
__device__ __forceinline__ float rnd(float v) {
    return to_f32<DT>(from_f32<DT>(v));
}

__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int DT, int NB, int RPW, int KMAX>
__global__ __launch_bounds__(LT) void rows_linear_kernel(RowsLinK a) {
    using st = typename Stor<DT>::type;
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [NB][K] in the storage type
    __shared__ float red[2][NB][LW];
    __shared__ unsigned long long best[NB][LW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int K = a.K, K8 = K / 8;

    // ---- for one or two batch rows the wave's first weight pieces are
    // requested before x is staged: they do not depend on it, so their latency
    // overlaps the LayerNorm (with more rows the staged pieces of x fill the
    // registers, and the early pieces would cost a wave per SIMD)
    constexpr bool PRE = NB <= 2 || (KMAX <= 1024 && RPW == 1);
    const int n0 = (blockIdx.x * LW + w) * RPW;
    const st *wr[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) wr[i] = (const st *)a.w + (int64_t)min(n0 + i, a.N - 1) * K;
    constexpr int U = 4;
    u32x4 wv0[PRE ? RPW : 1][U];
    if constexpr (PRE) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = min(lane + 64 * u, K8 - 1);
#pragma unroll
            for (int i = 0; i < RPW; ++i) wv0[i][u] = __builtin_nontemporal_load((const u32x4 *)(wr[i] + 8 * c));
        }
    }

    // ---- stage x (LayerNorm'd when ln_w is given) in LDS.  LayerNorm: every
    // 16-byte piece of the NB rows is loaded once into registers, the sums and
    // sums of squares of each row go through one block reduction, and the
    // normalised pieces are written with 16-byte LDS stores.
    if (a.ln_w) {
        constexpr int MAXP = (NB * KMAX / 8 + LT - 1) / LT;  // pieces per thread at K = KMAX
        const int np = NB * K8;
        u32x4 xp[MAXP];
        // Two passes over the register-held pieces: the mean first, then the
        // sum of squared deviations (no E[x^2] - mean^2 cancellation).
        float s1[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) s1[b] = 0.f;
#pragma unroll
        for (int j = 0; j < MAXP; ++j) {
            const int c = tid + LT * j;
            if (c < np) {
                const int b = c / K8, k8 = c % K8;
                xp[j] = *(const u32x4 *)((const st *)a.x + b * a.x_st + 8 * k8);
                float f[8];
                unpack16<DT>(xp[j], f);
                float t1 = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) t1 += f[e];
#pragma unroll
                for (int bb = 0; bb < NB; ++bb)
                    if (bb == b) s1[bb] += t1;
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float t1 = wave_sum(s1[b]);
            if (lane == 0) red[0][b][w] = t1;
        }
        __syncthreads();
        float mean[NB], rstd[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float t1 = 0.f;
#pragma unroll
            for (int i = 0; i < LW; ++i) t1 += red[0][b][i];
            mean[b] = t1 / (float)K;
            s1[b] = 0.f;
        }
#pragma unroll
        for (int j = 0; j < MAXP; ++j) {
            const int c = tid + LT * j;
            if (c < np) {
                const int b = c / K8;
                float mb = mean[0];
#pragma unroll
                for (int bb = 1; bb < NB; ++bb)
                    if (bb == b) mb = mean[bb];
                float f[8];
                unpack16<DT>(xp[j], f);
                float t2 = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) t2 = fmaf(f[e] - mb, f[e] - mb, t2);
#pragma unroll
                for (int bb = 0; bb < NB; ++bb)
                    if (bb == b) s1[bb] += t2;
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float t2 = wave_sum(s1[b]);
            if (lane == 0) red[1][b][w] = t2;
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float t2 = 0.f;
#pragma unroll
            for (int i = 0; i < LW; ++i) t2 += red[1][b][i];
            rstd[b] = rsqrtf(t2 / (float)K + a.ln_eps);
        }
#pragma unroll
        for (int j = 0; j < MAXP; ++j) {
            const int c = tid + LT * j;
            if (c < np) {
                const int b = c / K8, k8 = c % K8;
                float mb = mean[0], rb = rstd[0];
#pragma unroll
                for (int bb = 1; bb < NB; ++bb)
                    if (bb == b) {
                        mb = mean[bb];
                        rb = rstd[bb];
                    }
                float f[8], g[8], o[8];
                unpack16<DT>(xp[j], f);
                unpack16<DT>(*(const u32x4 *)((const st *)a.ln_w + 8 * k8), g);
                if (a.ln_b) {
                    unpack16<DT>(*(const u32x4 *)((const st *)a.ln_b + 8 * k8), o);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[e] = 0.f;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = fmaf((f[e] - mb) * rb, g[e], o[e]);
                *(u32x4 *)&xs[b * K + 8 * k8] = u32x4{pack2<DT>(o[0], o[1]), pack2<DT>(o[2], o[3]),
                                                      pack2<DT>(o[4], o[5]), pack2<DT>(o[6], o[7])};
            }
        }
    } else {
        for (int c = tid; c < NB * K8; c += LT) {
            const int b = c / K8, k8 = c % K8;
            *(u32x4 *)&xs[b * K + 8 * k8] = *(const u32x4 *)((const st *)a.x + b * a.x_st + 8 * k8);
        }
    }
    __syncthreads();

    // ---- RPW rows per wave, 16-byte weight pieces, four pieces in flight per row
    float acc[RPW][NB];
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[i][b] = 0.f;
    for (int c0 = lane; c0 < K8; c0 += 64 * U) {
        u32x4 wv[RPW][U];
        if (PRE && c0 == lane) {  // the pieces loaded before the staging
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int i = 0; i < RPW; ++i) wv[i][u] = wv0[PRE ? i : 0][u];
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = min(c0 + 64 * u, K8 - 1);
#pragma unroll
                for (int i = 0; i < RPW; ++i) wv[i][u] = __builtin_nontemporal_load((const u32x4 *)(wr[i] + 8 * c));
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + 64 * u;
            if (c < K8) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    float xv[8];
                    unpack16<DT>(*(const u32x4 *)&xs[b * K + 8 * c], xv);
#pragma unroll
                    for (int i = 0; i < RPW; ++i) {
                        float wf[8];
                        unpack16<DT>(wv[i][u], wf);
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc[i][b] = fmaf(wf[e], xv[e], acc[i][b]);
                    }
                }
            }
        }
    }

    // ---- reduce over the wave; lane i*NB+b finishes value (row i, batch b)
    float mine = 0.f;
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float t = wave_sum(acc[i][b]);
            if (lane == i * NB + b) mine = t;
        }
    const int i_me = lane / NB, b_me = lane % NB, n = n0 + i_me;
    unsigned long long key = 0ull;
    if (lane < RPW * NB && n < a.N) {
        float v = mine;
        if (a.bias) v += to_f32<DT>(((const st *)a.bias)[n]);
        v = rnd<DT>(v);
        if (a.act == 1) v = rnd<DT>(0.5f * v * (1.f + erff(v * 0.70710678118654752f)));
        if (n < a.scale_cols) v = rnd<DT>(v * a.scale);
        if (a.res) v = rnd<DT>(to_f32<DT>(((const st *)a.res)[b_me * a.res_st + n]) + v);
        ((st *)a.y)[b_me * a.y_st + n] = from_f32<DT>(v);
        key = ((unsigned long long)order_key(v) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)n);
    }
    if (a.argmax) {  // block-wide best key per batch row, written to the block's own slot
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            unsigned long long k = b_me == b && lane < RPW * NB ? key : 0ull;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const uint32_t lo = __shfl_xor((uint32_t)k, off), hi = __shfl_xor((uint32_t)(k >> 32), off);
                const unsigned long long o = ((unsigned long long)hi << 32) | lo;
                k = o > k ? o : k;
            }
            if (lane == 0) best[b][w] = k;
        }
        __syncthreads();
        if (tid < a.B) {  // one slot per (row, block): no atomics; the feedback kernel reduces the slots
            unsigned long long k = best[tid][0];
#pragma unroll
            for (int i = 1; i < LW; ++i) k = best[tid][i] > k ? best[tid][i] : k;
            a.argmax[(int64_t)tid * gridDim.x + blockIdx.x] = k;
        }
    }
}

template <int DT, int NB, int KMAX>
int launch_rows_k(const RowsLinK &k, hipStream_t s) {
    const size_t lds = (size_t)NB * k.K * 2;
    if (k.N >= 16384 || k.argmax) {  // argmax slots assume 16 rows per block
        constexpr int RPW = 4;
        hipLaunchKernelGGL((rows_linear_kernel<DT, NB, RPW, KMAX>), dim3((k.N + LW * RPW - 1) / (LW * RPW)),
                           dim3(LT), lds, s, k);
    } else {
        constexpr int RPW = 1;
        hipLaunchKernelGGL((rows_linear_kernel<DT, NB, RPW, KMAX>), dim3((k.N + LW * RPW - 1) / (LW * RPW)),
                           dim3(LT), lds, s, k);
    }
    return HOFA_OK;
}

// K <= 1024 (the attention and fc1 inputs of the cfg5 model) stages fewer
// LayerNorm pieces per thread, which leaves registers for the early weight loads.
template <int DT, int NB>
int launch_rows(const RowsLinK &k, hipStream_t s) {
    return k.K <= 1024 ? launch_rows_k<DT, NB, 1024>(k, s) : launch_rows_k<DT, NB, 4096>(k, s);
}

template <int DT>
int dispatch_rows(const RowsLinK &k, hipStream_t s) {
    switch (k.B) {
        case 1: return launch_rows<DT, 1>(k, s);
        case 2: return launch_rows<DT, 2>(k, s);
        case 3: return launch_rows<DT, 3>(k, s);
        default: return launch_rows<DT, 4>(k, s);
    }
}

// ------------------------------------------------------------------ prologue
struct PrologueK {
    void *qkv;
    const void *gate_w, *gate_b, *mix_w, *mix_b, *fixed_mix;
    const void *cos, *sin;
    const int64_t *pos;
    void *cache_k, *cache_v;
    float *log_gamma, *mix;
    int64_t qkv_st;
    int B, H, D, R, cache_len, rope_rows, rope, rope_dt;
};

template <int DT, int D>
__global__ __launch_bounds__(64) void decode_prologue_kernel(PrologueK a) {
    using st = typename Stor<DT>::type;
    constexpr int PL = D / 64;  // channels per lane: d = lane + 64 p
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H, lane = threadIdx.x;
    const int HD = a.H * D;
    st *qr = (st *)a.qkv + b * a.qkv_st + h * D;
    st *kr = qr + HD;
    const st *vr = qr + 2 * HD;
    float q[PL], k[PL];
    float gq = 0.f, gk = 0.f, mq = 0.f, mk = 0.f;
#pragma unroll
    for (int p = 0; p < PL; ++p) {
        const int d = lane + 64 * p;
        q[p] = to_f32<DT>(qr[d]);
        k[p] = to_f32<DT>(kr[d]);
        const st *gw = (const st *)a.gate_w + h * 2 * D;
        gq = fmaf(q[p], to_f32<DT>(gw[d]), gq);
        gk = fmaf(k[p], to_f32<DT>(gw[D + d]), gk);
        if (a.mix_w) {
            const st *mw = (const st *)a.mix_w + h * 2 * D;
            mq = fmaf(q[p], to_f32<DT>(mw[d]), mq);
            mk = fmaf(k[p], to_f32<DT>(mw[D + d]), mk);
        }
    }
    gq = wave_sum(gq);
    gk = wave_sum(gk);
    mq = wave_sum(mq);
    mk = wave_sum(mk);
    const int64_t pos = *a.pos;
    if (lane == 0) {
        // 16-bit logits as the module's ops produce them: each einsum rounded,
        // then their sum, then the sum with the bias; log_gamma =
        // logsigmoid(-gate) and mix = sigmoid(.) rounded likewise
        const float gl = rnd<DT>(rnd<DT>(rnd<DT>(gq) + rnd<DT>(gk)) + to_f32<DT>(((const st *)a.gate_b)[h]));
        const float ng = -gl;
        const float lg = fminf(ng, 0.f) - log1pf(expf(-fabsf(ng)));
        a.log_gamma[bh] = rnd<DT>(lg);
        float ml;
        if (a.mix_w) ml = rnd<DT>(rnd<DT>(rnd<DT>(mq) + rnd<DT>(mk)) + to_f32<DT>(((const st *)a.mix_b)[h]));
        else ml = to_f32<DT>(((const st *)a.fixed_mix)[h]);
        a.mix[bh] = rnd<DT>(1.f / (1.f + expf(-ml)));
    }
    // RoPE of channels [0, R) at row pos: x*cos + rotate_half(x)*sin.  With
    // 16-bit tables (a 16-bit module casts its RoPE buffers) each product is
    // rounded as the module's 16-bit ops round it; f32 tables round once.
    const int R = a.R, half = R / 2;
    if (a.rope) {
        const int64_t prow = min(pos, (int64_t)a.rope_rows - 1) * R;
        const float qp = __shfl(q[0], lane < half ? lane + half : lane - half);
        const float kp = __shfl(k[0], lane < half ? lane + half : lane - half);
        if (lane < R) {
            const float c = load_any(a.cos, a.rope_dt, prow + lane), s = load_any(a.sin, a.rope_dt, prow + lane);
            const float sg = lane < half ? -1.f : 1.f;
            if (a.rope_dt == HOFA_F32) {
                q[0] = rnd<DT>(q[0] * c + sg * qp * s);
                k[0] = rnd<DT>(k[0] * c + sg * kp * s);
            } else {
                q[0] = rnd<DT>(rnd<DT>(q[0] * c) + rnd<DT>(sg * qp * s));
                k[0] = rnd<DT>(rnd<DT>(k[0] * c) + rnd<DT>(sg * kp * s));
            }
            qr[lane] = from_f32<DT>(q[0]);
            kr[lane] = from_f32<DT>(k[0]);
        }
    }
    // cache append at row pos
    const int64_t row = min(pos, (int64_t)a.cache_len - 1);
    st *ck = (st *)a.cache_k + ((int64_t)bh * a.cache_len + row) * R;
    st *cv = (st *)a.cache_v + ((int64_t)bh * a.cache_len + row) * D;
    if (lane < R) ck[lane] = from_f32<DT>(k[0]);
#pragma unroll
    for (int p = 0; p < PL; ++p) cv[lane + 64 * p] = vr[lane + 64 * p];
}

// ------------------------------------------------------------------ advance
struct AdvanceK {
    const unsigned long long *argmax;  // [B][slots] per-block keys of the LM head
    const void *emb;
    void *x;
    int64_t *tok, *out, *col, *pos;
    int32_t *seq_len;
    int64_t x_st, out_st;
    int B, Dm, V, out_cols, slots;
};

template <int DT>
__global__ __launch_bounds__(256) void decode_advance_kernel(AdvanceK a) {
    using st = typename Stor<DT>::type;
    __shared__ unsigned long long s_best[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t col = *a.col;
    for (int b = 0; b < a.B; ++b) {
        // greatest key over the LM head's per-block slots of row b
        unsigned long long key = 0ull;
        for (int i = tid; i < a.slots; i += 256) {
            const unsigned long long k = a.argmax[(int64_t)b * a.slots + i];
            key = k > key ? k : key;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)key, off), hi = __shfl_xor((uint32_t)(key >> 32), off);
            const unsigned long long o = ((unsigned long long)hi << 32) | lo;
            key = o > key ? o : key;
        }
        if (lane == 0) s_best[w] = key;
        __syncthreads();
        key = s_best[0];
#pragma unroll
        for (int i = 1; i < 4; ++i) key = s_best[i] > key ? s_best[i] : key;
        __syncthreads();  // s_best is reused by the next row
        const int64_t idx = min((int64_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull)), (int64_t)a.V - 1);
        const st *er = (const st *)a.emb + idx * a.Dm;
        st *xr = (st *)a.x + b * a.x_st;
        for (int d = tid; d < a.Dm; d += 256) xr[d] = er[d];
        if (tid == 0) {
            a.tok[b] = idx;
            if (col < a.out_cols) a.out[b * a.out_st + col] = idx;
        }
    }
    __syncthreads();  // every counter read above happens before the writes below
    if (tid == 0) {
        *a.col = col + 1;
        *a.pos = *a.pos + 1;
        *a.seq_len = *a.seq_len + 1;
    }
}

}  // namespace
}  // namespace hofa

using namespace hofa;

extern "C" int hofa_rows_linear(const hofa_rows_linear_args_t *a, void *stream) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_rows_linear: args is NULL");
    HOFA_REQUIRE(a->B >= 1 && a->B <= 4, HOFA_EUNSUPPORTED, "hofa_rows_linear: B=%d not in [1, 4]", a->B);
    HOFA_REQUIRE(a->K > 0 && a->K % 8 == 0 && a->K <= 4096, HOFA_EUNSUPPORTED,
                 "hofa_rows_linear: K=%d must be a positive multiple of 8, at most 4096", a->K);
    HOFA_REQUIRE(a->N > 0, HOFA_EINVAL, "hofa_rows_linear: N=%d must be positive", a->N);
    HOFA_REQUIRE(a->dtype == HOFA_BF16 || a->dtype == HOFA_F16, HOFA_EUNSUPPORTED,
                 "hofa_rows_linear: dtype %d must be bf16 or f16", a->dtype);
    HOFA_REQUIRE(a->act == 0 || a->act == 1, HOFA_EINVAL, "hofa_rows_linear: act=%d not in {0, 1}", a->act);
    HOFA_REQUIRE(a->x && a->w && a->y, HOFA_EINVAL, "hofa_rows_linear: NULL x, w or y");
    HOFA_REQUIRE(a->ln_w || !a->ln_b, HOFA_EINVAL, "hofa_rows_linear: ln_b without ln_w");
    HOFA_REQUIRE(((uintptr_t)a->w % 16) == 0 && ((uintptr_t)a->x % 16) == 0 && a->x_stride % 8 == 0 &&
                     ((uintptr_t)a->ln_w % 16) == 0 && ((uintptr_t)a->ln_b % 16) == 0,
                 HOFA_EINVAL, "hofa_rows_linear: w, x, ln_w and ln_b must be 16-byte aligned rows");
    HOFA_REQUIRE(a->x_stride >= a->K && a->y_stride >= a->N && (!a->res || a->res_stride >= a->N), HOFA_EINVAL,
                 "hofa_rows_linear: row strides smaller than the row length");
    RowsLinK k{};
    k.x = a->x; k.ln_w = a->ln_w; k.ln_b = a->ln_b; k.w = a->w; k.bias = a->bias; k.res = a->res;
    k.y = a->y; k.argmax = a->argmax;
    k.x_st = a->x_stride; k.res_st = a->res_stride; k.y_st = a->y_stride;
    k.B = a->B; k.K = a->K; k.N = a->N; k.act = a->act; k.scale_cols = a->scale_cols;
    k.scale = a->scale; k.ln_eps = a->ln_eps;
    hipStream_t s = (hipStream_t)stream;
    if (a->dtype == HOFA_BF16) dispatch_rows<HOFA_BF16>(k, s);
    else dispatch_rows<HOFA_F16>(k, s);
    return check_launch("hofa_rows_linear");
}

extern "C" int hofa_decode_prologue(const hofa_decode_prologue_args_t *a, void *stream) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_decode_prologue: args is NULL");
    HOFA_REQUIRE(a->B > 0 && a->H > 0, HOFA_EINVAL, "hofa_decode_prologue: B=%d H=%d", a->B, a->H);
    HOFA_REQUIRE(a->D == 64 || a->D == 128, HOFA_EUNSUPPORTED, "hofa_decode_prologue: D=%d not in {64, 128}", a->D);
    HOFA_REQUIRE(a->R > 0 && a->R <= 64 && a->R % 2 == 0 && a->R < a->D, HOFA_EUNSUPPORTED,
                 "hofa_decode_prologue: R=%d must be even, in (0, 64] and below D", a->R);
    HOFA_REQUIRE(a->dtype == HOFA_BF16 || a->dtype == HOFA_F16, HOFA_EUNSUPPORTED,
                 "hofa_decode_prologue: dtype %d must be bf16 or f16", a->dtype);
    HOFA_REQUIRE(a->qkv && a->gate_w && a->gate_b && a->pos && a->cache_k && a->cache_v && a->log_gamma && a->mix,
                 HOFA_EINVAL, "hofa_decode_prologue: NULL pointer argument");
    HOFA_REQUIRE((a->mix_w && a->mix_b) || a->fixed_mix, HOFA_EINVAL,
                 "hofa_decode_prologue: need mix_w and mix_b, or fixed_mix");
    HOFA_REQUIRE(!a->cos == !a->sin && (!a->cos || a->rope_rows > 0), HOFA_EINVAL,
                 "hofa_decode_prologue: cos and sin go together, with rope_rows > 0");
    HOFA_REQUIRE(!a->cos || a->rope_dtype == HOFA_F32 || a->rope_dtype == a->dtype, HOFA_EINVAL,
                 "hofa_decode_prologue: rope_dtype %d must be f32 or the qkv dtype", a->rope_dtype);
    HOFA_REQUIRE(a->cache_len > 0 && a->qkv_stride >= 3 * a->H * a->D, HOFA_EINVAL,
                 "hofa_decode_prologue: cache_len=%d, qkv_stride=%lld", a->cache_len, (long long)a->qkv_stride);
    PrologueK k{};
    k.qkv = a->qkv; k.gate_w = a->gate_w; k.gate_b = a->gate_b; k.mix_w = a->mix_w; k.mix_b = a->mix_b;
    k.fixed_mix = a->fixed_mix; k.cos = a->cos; k.sin = a->sin; k.pos = a->pos;
    k.cache_k = a->cache_k; k.cache_v = a->cache_v; k.log_gamma = a->log_gamma; k.mix = a->mix;
    k.qkv_st = a->qkv_stride;
    k.B = a->B; k.H = a->H; k.D = a->D; k.R = a->R; k.cache_len = a->cache_len; k.rope_rows = a->rope_rows;
    k.rope = a->cos != nullptr;
    k.rope_dt = a->rope_dtype;
    hipStream_t s = (hipStream_t)stream;
    const dim3 g(a->B * a->H), t(64);
    if (a->dtype == HOFA_BF16) {
        if (a->D == 64) hipLaunchKernelGGL((decode_prologue_kernel<HOFA_BF16, 64>), g, t, 0, s, k);
        else hipLaunchKernelGGL((decode_prologue_kernel<HOFA_BF16, 128>), g, t, 0, s, k);
    } else {
        if (a->D == 64) hipLaunchKernelGGL((decode_prologue_kernel<HOFA_F16, 64>), g, t, 0, s, k);
        else hipLaunchKernelGGL((decode_prologue_kernel<HOFA_F16, 128>), g, t, 0, s, k);
    }
    return check_launch("hofa_decode_prologue");
}

extern "C" int hofa_decode_advance(const hofa_decode_advance_args_t *a, void *stream) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_decode_advance: args is NULL");
    HOFA_REQUIRE(a->B >= 1 && a->B <= 4, HOFA_EUNSUPPORTED, "hofa_decode_advance: B=%d not in [1, 4]", a->B);
    HOFA_REQUIRE(a->d_model > 0 && a->vocab > 0 && a->out_cols > 0, HOFA_EINVAL,
                 "hofa_decode_advance: d_model=%d vocab=%d out_cols=%d", a->d_model, a->vocab, a->out_cols);
    HOFA_REQUIRE(a->dtype == HOFA_BF16 || a->dtype == HOFA_F16, HOFA_EUNSUPPORTED,
                 "hofa_decode_advance: dtype %d must be bf16 or f16", a->dtype);
    HOFA_REQUIRE(a->argmax && a->emb && a->x && a->tok && a->out && a->col && a->pos && a->seq_len, HOFA_EINVAL,
                 "hofa_decode_advance: NULL pointer argument");
    AdvanceK k{};
    k.argmax = a->argmax; k.emb = a->emb; k.x = a->x; k.tok = a->tok; k.out = a->out; k.col = a->col;
    k.pos = a->pos; k.seq_len = a->seq_len; k.x_st = a->x_stride; k.out_st = a->out_stride;
    k.B = a->B; k.Dm = a->d_model; k.V = a->vocab; k.out_cols = a->out_cols;
    k.slots = (a->vocab + 15) / 16;
    hipStream_t s = (hipStream_t)stream;
    if (a->dtype == HOFA_BF16) hipLaunchKernelGGL((decode_advance_kernel<HOFA_BF16>), dim3(1), dim3(256), 0, s, k);
    else hipLaunchKernelGGL((decode_advance_kernel<HOFA_F16>), dim3(1), dim3(256), 0, s, k);
    return check_launch("hofa_decode_advance");
}

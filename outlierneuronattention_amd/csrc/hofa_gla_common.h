// Pieces shared by the chunked GLA forward (hofa_gla.hip) and backward
// (hofa_gla_bwd.hip): chunk constants, the in-chunk decay cumsum, two-phase
// (issue, then commit) transposed LDS staging, and the per-chunk
// outer-product kernel used by both passes
// (forward: dS^T = V^T (K (.) exp(G_last - G)); backward: dH^T = dO^T (Q (.) exp(G))).
#pragma once

#include "hofa_mfma.h"

namespace hofa {
namespace gla {

constexpr int C = 64;               // chunk length
constexpr float kSafeRange = 64.f;  // max in-chunk -G for factored exp(+-G) operands (exp(64) ~ 6e27)

// Every GLA matrix product takes bf16 operands (the f32 exponent range keeps
// the factored exp(+-G) operands finite); f32 and f16 inputs are split into a
// bf16 hi/lo pair (exact for f16), bf16 inputs are used as they are.
constexpr int OPB = HOFA_BF16;
template <int DT> constexpr bool kRawSplit = DT != HOFA_BF16;

// The T rows of one head's [T, *] operand through a range-checked buffer:
// rows at or past T read as zeros, so tile loads need no branches.  The
// base pointer must be wave-uniform; the host checks that (T + 2C) rows span
// less than 2 GiB.
template <int DT>
struct Rows {
    using in_t = typename Stor<DT>::type;
    __amdgpu_buffer_rsrc_t r;
    int64_t st;
    __device__ Rows(const in_t *base, int64_t row_stride, int T)
        : r(rows_rsrc(base, (uint32_t)(T * row_stride * (int64_t)sizeof(in_t)))), st(row_stride) {}
    __device__ uint32_t off(int row, int col) const { return (uint32_t)((row * st + col) * (int64_t)sizeof(in_t)); }
};

// Four consecutive outputs (16-byte aligned for f32, 8-byte for 16-bit types).
template <int DT>
__device__ __forceinline__ void store4(typename Stor<DT>::type *p, float a, float b, float c, float d) {
    if constexpr (DT == HOFA_F32) {
        *(f32x4 *)p = f32x4{a, b, c, d};
    } else {
        *(uint2 *)p = uint2{pack2<DT>(a, b), pack2<DT>(c, d)};
    }
}

// Where a chunk kernel finds its inputs.  Forward and backward fill the
// fields they use; strides are in elements.
struct GlaK {
    const void *q, *k, *v, *lg, *la, *g, *mix, *gs;
    void *y;
    void *n_out;        // optional RMSNorm(Y_I) before the gate (forward)
    float *rstd;        // optional 1/sqrt(mean(Y_I^2)+eps) per token (forward)
    float *state_out;
    float *ws_ds;       // [B*H][nc][D][J] f32 per-chunk outer products
    float *ws_gl;       // [B*H][nc][J] f32 per-chunk total log decay
    uint16_t *s_in;     // [B*H][nc][nplanes][D*J] entering states as 16-bit planes
    uint8_t *unsafe;    // [B*H*nc] per chunk: decay range beyond kSafeRange (set by gla_state_kernel)
    int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, y_sb, y_sh, y_st;
    int64_t n_sb, n_sh, n_st;
    int64_t lg_sb, lg_sh, lg_st, la_sh, la_sj, g_sb, g_sh, g_st, g_sj;
    int64_t m_sb, m_sh, m_st, gs_sh, gs_sd;
    int64_t so_sb, so_sh, so_sj, so_sd;
    int lg_dt, la_dt, mix_dt, gs_dt;
    int B, H, T, R, nc;
    int key_col0;       // first column of the key operand of gla_state_kernel
    int nplanes;        // 1: bf16 S^T [D][J]; 2: hi/lo of S^T; 4: also hi/lo of S [J][D]
    int pad_rows;       // state_out rows J .. J+pad_rows-1 to write as zeros
    int fuse;
    int y_f32;          // y is float32 (unrounded result) rather than the input dtype
    float eps;
};

// In-chunk inclusive cumsum G[t][c] of the log decay (t < C, c < J), in LDS.
// Scalar decay keeps two vectors and forms G = Lambda[t] * alpha[c] on the fly
// (Lambda = in-chunk cumsum of log_gamma, alpha = exp(log_alpha)); general
// decay keeps a [C][J+1] table, the odd pitch spreading lane-per-token reads
// over all banks.  Tokens past T decay by 0.  Eight trailing floats hold the
// per-wave partial maxima behind range().
template <int J, bool GENERAL>
struct Decay {
    static constexpr int GP = J + 1;
    static constexpr int kBody = GENERAL ? C * GP : C + J;
    static constexpr int kFloats = kBody + 8;
    float *s;
    __device__ __forceinline__ float G(int t, int c) const {
        if constexpr (GENERAL) return s[t * GP + c];
        else return s[t] * s[C + c];
    }
    __device__ __forceinline__ float last(int c) const { return G(C - 1, c); }
    // Largest |G| over the chunk (valid after DecayStage::commit).
    __device__ __forceinline__ float range() const {
        const float *r = s + kBody;
        if constexpr (GENERAL) return fmaxf(fmaxf(r[0], r[1]), fmaxf(r[2], r[3]));
        else return r[0] * r[1];
    }
};

// ---- two-phase staging: issue() starts a tile's global loads into registers,
// commit() writes it to LDS later, so that the loads of every tile of a chunk
// are in flight together instead of one tile per barrier.

// The 16-byte vectors holding 8 consecutive input elements (two for f32).
template <int DT>
struct Raw8 {
    static constexpr int NV = DT == HOFA_F32 ? 2 : 1;
    u32x4 w[NV];
    __device__ __forceinline__ void load(const Rows<DT> &rows, int row, int col) {
        w[0] = bload16(rows.r, rows.off(row, col));
        if constexpr (NV == 2) w[1] = bload16(rows.r, rows.off(row, col) + 16);
    }
    __device__ __forceinline__ void get(float *x) const {
        if constexpr (NV == 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[e] = __uint_as_float(w[0][e]);
                x[4 + e] = __uint_as_float(w[1][e]);
            }
        } else {
            unpack16<DT>(w[0], x);
        }
    }
};

// Token-granule swizzle of a transposed tile: element (row, t) at
// row * PITCH + ((t / 8) ^ tr_swz(row)) * 8 + t % 8.  With PITCH = 8 (mod 16),
// a commit's 4-byte stores to rows eight channels apart (a [64][PITCH] tile
// store pass) fall on distinct banks instead of four rows per bank, and reads
// of 16 consecutive rows at one token granule (tr_swz constant over them)
// stay conflict-free.
__device__ __forceinline__ int tr_swz(int row) { return 2 * ((row >> 4) & 3); }

// Column swizzle of the transposed V tile of gla_out_kernel (PITCH = 4 mod
// 16): token t of row r at column t ^ (16 if r % 64 >= 32), so the commit
// stores of rows 32 channels apart fall on different banks; the output
// kernel's 8-byte operand reads of 32 consecutive rows stay conflict-free.
__device__ __forceinline__ int tr_col_swz(int row) { return ((row >> 5) & 1) << 4; }

// A [C x W] chunk tile (columns [col0, col0+W)) in pieces of 2 rows x 8
// columns per thread, committed to LDS transposed ([W][PITCH] 16-bit
// operands, tokens contiguous); rows past T are zero.  SWZ = 1: token
// granules swizzled by tr_swz; SWZ = 2: columns swizzled by tr_col_swz.
template <int DT, int W, int NTH, int SWZ = 0>
struct TrStage {
    static constexpr int NPIECE = (C / 2) * (W / 8);
    static constexpr int PT = (NPIECE + NTH - 1) / NTH;
    Raw8<DT> raw[PT][2];
    __device__ __forceinline__ void issue(const Rows<DT> &rows, int col0, int t0) {
#pragma unroll
        for (int p = 0; p < PT; ++p) {
            const int pi = threadIdx.x + p * NTH;
            if (NPIECE % NTH == 0 || pi < NPIECE) {
                const int tp = pi / (W / 8), cc = pi % (W / 8);
                raw[p][0].load(rows, t0 + 2 * tp, col0 + 8 * cc);
                raw[p][1].load(rows, t0 + 2 * tp + 1, col0 + 8 * cc);
            }
        }
    }
    // Element (t, ch) of the tile is multiplied by scale(t, ch); with LO the
    // bf16 rounding remainder goes to dst_lo.
    template <int PITCH, bool LO, typename Scale>
    __device__ __forceinline__ void commit(uint16_t *dst, uint16_t *dst_lo, Scale scale) const {
#pragma unroll
        for (int p = 0; p < PT; ++p) {
            const int pi = threadIdx.x + p * NTH;
            if (NPIECE % NTH == 0 || pi < NPIECE) {
                const int tp = pi / (W / 8), cc = pi % (W / 8);
                const int t = 2 * tp;
                float x[2][8];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    raw[p][r].get(x[r]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[r][e] *= scale(t + r, 8 * cc + e);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int row = 8 * cc + e;
                    const int o = SWZ == 1   ? row * PITCH + (((t >> 3) ^ tr_swz(row)) << 3) + (t & 7)
                                  : SWZ == 2 ? row * PITCH + (t ^ tr_col_swz(row))
                                             : row * PITCH + t;
                    const uint32_t hv = pack2<OPB>(x[0][e], x[1][e]);
                    *(uint32_t *)&dst[o] = hv;
                    if constexpr (LO)
                        *(uint32_t *)&dst_lo[o] = pack2<OPB>(x[0][e] - op_to_f32<OPB>(hv & 0xffffu),
                                                             x[1][e] - op_to_f32<OPB>(hv >> 16));
                }
            }
        }
    }
};

// The decay of chunk [t0, t0+C) of head (b, h): issue() loads it into
// registers, commit() fills a Decay (ends with a barrier).  NTH threads,
// 128 <= NTH <= 256.
template <int J, bool GENERAL, int NTH>
struct DecayStage {
    static_assert(NTH >= 128 && NTH <= 256, "two to four waves");
    static constexpr int NW = NTH / 64;
    static constexpr int NG = GENERAL ? (C * J / 4 + NTH - 1) / NTH : 1;
    static constexpr int NA = (J + 63) / 64;
    f32x4 gv[NG];  // general: float4 pieces idx = tid + i NTH of the [C][J] tile
    float lgv;     // scalar decay, wave 0: log_gamma of token t0 + lane
    float lav[NA]; // scalar decay, wave 1: log_alpha of channel lane + 64 i
    __device__ __forceinline__ void issue(const GlaK &a, int b, int h, int t0) {
        const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
        if constexpr (!GENERAL) {
            if (w == 0) {
                const int t = t0 + lane;
                lgv = t < a.T ? load_any(a.lg, a.lg_dt, b * a.lg_sb + h * a.lg_sh + (int64_t)t * a.lg_st) : 0.f;
            } else if (w == 1) {
#pragma unroll
                for (int i = 0; i < NA; ++i) {
                    const int ch = lane + 64 * i;
                    lav[i] = a.la && ch < J ? load_any(a.la, a.la_dt, h * a.la_sh + ch * a.la_sj) : 0.f;
                }
            }
        } else {
            const float *gp = (const float *)a.g + b * a.g_sb + h * a.g_sh;
            const bool vec = a.g_sj == 1 && (a.g_st % 4) == 0 && (a.g_sb % 4) == 0 && (a.g_sh % 4) == 0 &&
                             ((uintptr_t)a.g % 16) == 0;
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                const int idx = tid + i * NTH;
                const int t = idx / (J / 4), c = 4 * (idx % (J / 4));
                f32x4 x = {0.f, 0.f, 0.f, 0.f};
                if ((C * J / 4) % NTH == 0 || idx < C * J / 4) {
                    if (t0 + t < a.T) {
                        const float *p = gp + (int64_t)(t0 + t) * a.g_st;
                        if (vec) {
                            x = *(const f32x4 *)(p + c);
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e) x[e] = p[(c + e) * a.g_sj];
                        }
                    }
                }
                gv[i] = x;
            }
        }
    }
    __device__ __forceinline__ void commit(const GlaK &a, Decay<J, GENERAL> dec) const {
        float *s = dec.s, *red = s + Decay<J, GENERAL>::kBody;
        const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
        if constexpr (!GENERAL) {
            if (w == 0) {
                const float x = wave_incl_scan(lgv);
                s[lane] = x;
                const float m = wave_max(fabsf(x));
                if (lane == 0) red[0] = m;
            } else if (w == 1) {
                float m = 0.f;
#pragma unroll
                for (int i = 0; i < NA; ++i) {
                    const int ch = lane + 64 * i;
                    if (ch < J) {
                        const float al = a.la ? expf(lav[i]) : 1.f;
                        s[C + ch] = al;
                        m = fmaxf(m, al);
                    }
                }
                m = wave_max(m);
                if (lane == 0) red[1] = m;
            }
            __syncthreads();
        } else {
            constexpr int GP = Decay<J, GENERAL>::GP;
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                const int idx = tid + i * NTH;
                if ((C * J / 4) % NTH == 0 || idx < C * J / 4) {
                    const int t = idx / (J / 4), c = 4 * (idx % (J / 4));
#pragma unroll
                    for (int e = 0; e < 4; ++e) s[t * GP + c + e] = gv[i][e];
                }
            }
            if (tid < 4) red[tid] = 0.f;
            __syncthreads();
            float m = 0.f;
            constexpr int NCOL = (J + NW - 1) / NW;
            float x[NCOL];
#pragma unroll
            for (int i = 0; i < NCOL; ++i) {  // columns w, w + NW, ..: lane = token
                const int c = w + i * NW;
                x[i] = J % NW == 0 || c < J ? s[lane * GP + c] : 0.f;
            }
#pragma unroll
            for (int i = 0; i < NCOL; ++i) x[i] = wave_incl_scan(x[i]);  // independent chains interleave
#pragma unroll
            for (int i = 0; i < NCOL; ++i) {
                const int c = w + i * NW;
                if (J % NW == 0 || c < J) {
                    s[lane * GP + c] = x[i];
                    m = fmaxf(m, fabsf(x[i]));
                }
            }
            m = wave_max(m);
            if (lane == 0) red[w] = m;
            __syncthreads();
        }
    }
};

// A backward pass (chunk_states, four planes per chunk) with D = 64 stages
// the S^T planes in LDS and reads S there with transposing loads, so only
// planes 0/1 are written; D = 128 reads all four planes from memory.
template <int D, int J> constexpr bool kStateLds = D == 64 && J <= 64;
template <int D, int J>
__host__ __device__ constexpr int planes_written(int nplanes) { return nplanes == 4 && kStateLds<D, J> ? 2 : nplanes; }

constexpr int kStateThreads = 256;  // four waves: the LDS footprint allows four blocks per CU

// Per chunk: in-chunk cumsum G of the log decay, then
//   forward (BWD=false): out^T[D x J] = V_c^T (K_c (.) exp(G_last - G))
//   backward (BWD=true): out^T[D x J] = dO_c^T (Q_c (.) exp(G))
// with the key operand read at columns [key_col0, key_col0+J) of a.k and the
// value operand from a.v (every exponent <= 0).  Writes out^T to ws_ds and
// G_last to ws_gl, and whether the chunk's decay range exceeds kSafeRange to
// unsafe[].  4 waves, v_mfma_f32_16x16x32 tiles.  The global loads of the
// decay, key and value tiles are all issued before the first barrier.  RND:
// the decayed key operand is rounded to bf16 once (the reference's
// K_c_decayed, src/chunk_gla_inlier.py:118-121); otherwise it is a hi/lo pair.
template <int DT, int D, int J, bool GENERAL, bool BWD, bool RND = false>
__global__ __launch_bounds__(kStateThreads) void gla_state_kernel(GlaK a) {
    using in_t = typename Stor<DT>::type;
    constexpr int NTH = kStateThreads;
    constexpr int TP = C + 8;                       // token pitch of the transposed tiles
    constexpr bool KLO = !RND;                      // key operand as a hi/lo pair
    constexpr bool VLO = kRawSplit<DT> && !RND;     // f32/f16 inputs also split the value operand
    __shared__ float sDec[Decay<J, GENERAL>::kFloats];
    __shared__ __attribute__((aligned(16))) uint16_t sKt[KLO ? 2 : 1][J * TP];
    __shared__ __attribute__((aligned(16))) uint16_t sVt[VLO ? 2 : 1][D * TP];
    const int bh = blockIdx.x / a.nc, c = blockIdx.x % a.nc;
    const int b = bh / a.H, h = bh % a.H, t0 = c * C;
    const Rows<DT> krows((const in_t *)a.k + b * a.k_sb + h * a.k_sh, a.k_st, a.T);
    const Rows<DT> vrows((const in_t *)a.v + b * a.v_sb + h * a.v_sh, a.v_st, a.T);
    DecayStage<J, GENERAL, NTH> dst;
    TrStage<DT, J, NTH, 1> kst;
    TrStage<DT, D, NTH, 1> vst;
    dst.issue(a, b, h, t0);
    kst.issue(krows, a.key_col0, t0);
    vst.issue(vrows, 0, t0);
    const Decay<J, GENERAL> dec{sDec};
    dst.commit(a, dec);
    if (threadIdx.x == 0) a.unsafe[blockIdx.x] = dec.range() > kSafeRange;
    if constexpr (BWD)
        kst.template commit<TP, KLO>(sKt[0], sKt[KLO ? 1 : 0],
                                     [&](int t, int ch) { return fast_exp2(dec.G(t, ch) * kLog2e); });
    else
        kst.template commit<TP, KLO>(sKt[0], sKt[KLO ? 1 : 0], [&](int t, int ch) {
            return fast_exp2((dec.last(ch) - dec.G(t, ch)) * kLog2e);
        });
    vst.template commit<TP, VLO>(sVt[0], sVt[VLO ? 1 : 0], [](int, int) { return 1.f; });
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r16 = lane & 15, g4 = lane >> 4;
    float *ds = a.ws_ds + ((int64_t)bh * a.nc + c) * D * J;
    constexpr int NTILE = (D / 16) * (J / 16);
    for (int tile = w; tile < NTILE; tile += NTH / 64) {
        const int tm = tile / (J / 16), tn = tile % (J / 16);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < C / 32; ++ks) {  // token granule 4 ks + g4 of rows 16 tm + r16 / 16 tn + r16
            const int vo = (16 * tm + r16) * TP + (((4 * ks + g4) ^ tr_swz(16 * tm)) << 3);
            const int ko = (16 * tn + r16) * TP + (((4 * ks + g4) ^ tr_swz(16 * tn)) << 3);
            const u32x4 av = *(const u32x4 *)&sVt[0][vo];
            acc = mfma16<OPB>(av, *(const u32x4 *)&sKt[0][ko], acc);
            if constexpr (KLO) acc = mfma16<OPB>(av, *(const u32x4 *)&sKt[KLO ? 1 : 0][ko], acc);
            if constexpr (VLO) acc = mfma16<OPB>(*(const u32x4 *)&sVt[VLO ? 1 : 0][vo], *(const u32x4 *)&sKt[0][ko], acc);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) ds[(16 * tm + 4 * g4 + v) * J + 16 * tn + r16] = acc[v];
    }
    for (int ch = threadIdx.x; ch < J; ch += NTH) a.ws_gl[((int64_t)bh * a.nc + c) * J + ch] = dec.last(ch);
}

// hi/lo 16-bit planes of 4 consecutive floats.
__device__ __forceinline__ void split4(const f32x4 &s, uint2 &hv, uint2 &lv) {
    hv = uint2{pack2<OPB>(s[0], s[1]), pack2<OPB>(s[2], s[3])};
    lv = uint2{pack2<OPB>(s[0] - op_to_f32<OPB>(hv.x & 0xffffu), s[1] - op_to_f32<OPB>(hv.x >> 16)),
               pack2<OPB>(s[2] - op_to_f32<OPB>(hv.y & 0xffffu), s[3] - op_to_f32<OPB>(hv.y >> 16))};
}

// Store the state elements (dv, j4..j4+3) of S^T ([D][J], j contiguous) as
// plane 0 (bf16 rounding) and, with two or more planes, plane 1 (remainder).
__device__ __forceinline__ void store_state_planes(uint16_t *dst, int nplanes, int D, int J, int dv, int j4,
                                                   const f32x4 &S) {
    uint2 hv, lv;
    split4(S, hv, lv);
    *(uint2 *)(dst + dv * J + j4) = hv;
    if (nplanes >= 2) *(uint2 *)(dst + D * J + dv * J + j4) = lv;
}

// The scans run one block per (head, kScanRows value rows) with thread
// (dvl, j4) carrying S[j4..j4+3][dv0 + dvl]; kScanRows * J / 4 threads.
constexpr int kScanRows = 16;
constexpr int kScanPitch = kScanRows + 4;  // LDS row pitch: 8-byte aligned rows, spread banks

// Store one chunk's state from a scan block: planes 0 (and 1) of S^T
// directly; with four planes, planes 2/3 (S, d contiguous) through the LDS tile
// sT[2][J * kScanPitch] (hi, lo), so that they also leave with contiguous
// stores.  Contains a barrier when nplanes == 4 (block-uniform); callers
// alternate between two tiles, so one barrier per chunk suffices.
template <int DT, int D, int J>
__device__ __forceinline__ void store_state_tile(uint16_t *dst, int nplanes, int dv0, int dvl, int j4,
                                                 const f32x4 &S, uint16_t *th, uint16_t *tl) {
    store_state_planes(dst, nplanes, D, J, dv0 + dvl, j4, S);
    if (nplanes != 4) return;
    uint2 hv, lv;
    split4(S, hv, lv);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t hb = e < 2 ? hv.x : hv.y, lb = e < 2 ? lv.x : lv.y;
        th[(j4 + e) * kScanPitch + dvl] = (uint16_t)((e & 1) ? hb >> 16 : hb & 0xffffu);
        tl[(j4 + e) * kScanPitch + dvl] = (uint16_t)((e & 1) ? lb >> 16 : lb & 0xffffu);
    }
    __syncthreads();  // the other tile was last read before the previous barrier
    const int tid = threadIdx.x;
    const int j = tid / (kScanRows / 4), c4 = (tid % (kScanRows / 4)) * 4;
    *(uint2 *)(dst + 2 * D * J + j * D + dv0 + c4) = *(const uint2 *)&th[j * kScanPitch + c4];
    *(uint2 *)(dst + 3 * D * J + j * D + dv0 + c4) = *(const uint2 *)&tl[j * kScanPitch + c4];
}

}  // namespace gla
}  // namespace hofa

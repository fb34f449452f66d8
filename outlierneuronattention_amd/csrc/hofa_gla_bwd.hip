// C entry point of the GLA + epilogue backward (kernels in hofa_gla_bwd_kernels.h).
#include "hofa_gla_bwd_kernels.h"

namespace hofa {
namespace glabwd {

// Instantiated in hofa_gla_bwd_inst.hip, one object per (dtype, head dim).
#define HOFA_GLA_BWD_EXTERN(DT, D)                                                    \
    extern template int launch_d<DT, D, false>(const GlaBwdK &, int, hipStream_t); \
    extern template int launch_d<DT, D, true>(const GlaBwdK &, int, hipStream_t);
HOFA_GLA_BWD_FOR_EACH(HOFA_GLA_BWD_EXTERN)
#undef HOFA_GLA_BWD_EXTERN

namespace {

// ------------------------------------------------------------------ host
int elem_bytes(int dt) { return dt == HOFA_F32 ? 4 : 2; }

bool rows_ok(const hofa_view_t &v, int es) {
    return v.stride[3] == 1 && ((uintptr_t)v.data % 16) == 0 && (v.stride[0] * es) % 16 == 0 &&
           (v.stride[1] * es) % 16 == 0 && (v.stride[2] * es) % 16 == 0;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct WsLayout {
    size_t dO, dh, gl, dse, dlg, cp, dgs, pla, pgs, flags, total;
};

WsLayout ws_layout(const hofa_gla_bwd_args_t *a) {
    const size_t bh = (size_t)a->B * a->H, T = a->T, D = a->D, J = a->D - a->R;
    const size_t nc = (T + C - 1) / C, ntile = (T + ET - 1) / ET;
    WsLayout w{};
    w.dO = 0;
    w.dh = w.dO + align256(bh * T * D * elem_bytes(a->q.dtype));
    w.gl = w.dh + align256(bh * nc * D * J * 4);
    w.dse = w.gl + align256(bh * nc * J * 4);
    w.dlg = w.dse + align256(bh * nc * 4 * D * J * 2);
    w.cp = w.dlg + align256(bh * T * 4);
    w.dgs = w.cp + align256(bh * nc * (2 * J + 2) * 4);
    w.pla = w.dgs + align256(bh * ntile * D * 4);
    w.pgs = w.pla + align256(bh * J * 4);
    w.flags = w.pgs + align256(bh * D * 4);
    w.total = w.flags + align256(bh * nc);
    return w;
}

int validate(const hofa_gla_bwd_args_t *a) {
    HOFA_REQUIRE(a, HOFA_EINVAL, "hofa_gla_bwd: args is NULL");
    HOFA_REQUIRE(a->B > 0 && a->H > 0 && a->T > 0, HOFA_EINVAL, "hofa_gla_bwd: B=%d H=%d T=%d must be positive", a->B,
                 a->H, a->T);
    HOFA_REQUIRE(a->T <= C * kMaxChunks, HOFA_EUNSUPPORTED, "hofa_gla_bwd: T=%d exceeds %d", a->T, C * kMaxChunks);
    HOFA_REQUIRE(a->D == 64 || a->D == 128, HOFA_EUNSUPPORTED, "hofa_gla_bwd: head dim D=%d not in {64,128}", a->D);
    const int J = a->D - a->R;
    HOFA_REQUIRE(a->R >= 0 && J >= 16 && J % 16 == 0, HOFA_EUNSUPPORTED,
                 "hofa_gla_bwd: inlier width J=%d must be a positive multiple of 16", J);
    const int dt = a->q.dtype;
    HOFA_REQUIRE(dt == HOFA_F32 || dt == HOFA_BF16 || dt == HOFA_F16, HOFA_EINVAL, "hofa_gla_bwd: bad dtype %d", dt);
    const int es = elem_bytes(dt);
    for (const hofa_view_t *v : {&a->q, &a->k, &a->v, &a->n, &a->dy, &a->dq, &a->dk, &a->dv}) {
        HOFA_REQUIRE(v->data, HOFA_EINVAL, "hofa_gla_bwd: NULL tensor pointer");
        HOFA_REQUIRE(v->dtype == dt, HOFA_EINVAL, "hofa_gla_bwd: q, k, v, n, dy, dq, dk, dv must share one dtype");
        HOFA_REQUIRE(rows_ok(*v, es), HOFA_EINVAL, "hofa_gla_bwd: tensors need unit last stride and 16-byte aligned rows");
    }
    for (const hofa_view_t *v : {&a->o, &a->dout_attn}) {
        if (!v->data) continue;
        HOFA_REQUIRE(v->dtype == dt && rows_ok(*v, es), HOFA_EINVAL,
                     "hofa_gla_bwd: o and dout_attn need the dtype of q and aligned rows");
    }
    HOFA_REQUIRE((a->R * es) % 16 == 0, HOFA_EINVAL, "hofa_gla_bwd: the inlier columns must start 16-byte aligned");
    for (const hofa_view_t *v : {&a->q, &a->k, &a->v, &a->dy, &a->n, &a->o}) {
        if (!v->data) continue;
        HOFA_REQUIRE((int64_t)(a->T + 2 * C) * v->stride[2] * es < (1ll << 31) &&
                         (int64_t)(a->T + 2 * C) * a->D * es < (1ll << 31),
                     HOFA_EUNSUPPORTED, "hofa_gla_bwd: one head's rows must span less than 2 GiB");
    }
    HOFA_REQUIRE(a->rstd && a->chunk_states && ((uintptr_t)a->chunk_states % 16) == 0, HOFA_EINVAL,
                 "hofa_gla_bwd: rstd and 16-byte aligned chunk_states from the forward are required");
    HOFA_REQUIRE(a->gla_scale.data && a->d_gla_scale.data, HOFA_EINVAL, "hofa_gla_bwd: gla_scale and d_gla_scale are required");
    if (a->g.data) {
        HOFA_REQUIRE(a->g.dtype == HOFA_F32 && a->d_g.data && a->d_g.dtype == HOFA_F32, HOFA_EINVAL,
                     "hofa_gla_bwd: general decay needs float32 g and d_g");
    } else {
        HOFA_REQUIRE(a->log_gamma.data && a->d_log_gamma.data, HOFA_EINVAL,
                     "hofa_gla_bwd: give log_gamma and d_log_gamma (or g and d_g)");
    }
    HOFA_REQUIRE(!a->d_log_alpha.data || (a->log_alpha.data && !a->g.data), HOFA_EINVAL,
                 "hofa_gla_bwd: d_log_alpha needs log_alpha and scalar decay");
    HOFA_REQUIRE(!a->d_mix.data || a->mix.data, HOFA_EINVAL, "hofa_gla_bwd: d_mix needs mix");
    HOFA_REQUIRE(!a->delta || a->o.data, HOFA_EINVAL, "hofa_gla_bwd: delta needs o");
    return HOFA_OK;
}

template <int DT, bool GEN>
int dispatch(const GlaBwdK &k, int D, int J, hipStream_t s) {
    return D == 64 ? launch_d<DT, 64, GEN>(k, J, s) : launch_d<DT, 128, GEN>(k, J, s);
}

}  // namespace
}  // namespace glabwd
}  // namespace hofa

using namespace hofa;
using namespace hofa::glabwd;

extern "C" size_t hofa_gla_bwd_workspace_bytes(const hofa_gla_bwd_args_t *a) {
    if (validate(a)) return 0;
    return ws_layout(a).total;
}

extern "C" int hofa_gla_bwd(const hofa_gla_bwd_args_t *a, void *workspace, size_t workspace_bytes, void *stream) {
    int rc = validate(a);
    if (rc) return rc;
    const WsLayout L = ws_layout(a);
    HOFA_REQUIRE(workspace && workspace_bytes >= L.total, HOFA_EWORKSPACE,
                 "hofa_gla_bwd: workspace of %zu bytes needed, got %zu", L.total, workspace_bytes);
    HOFA_REQUIRE(((uintptr_t)workspace % 256) == 0, HOFA_EWORKSPACE, "hofa_gla_bwd: workspace must be 256-byte aligned");
    GlaBwdK k{};
    GlaK &f = k.f;
    f.q = a->q.data; f.k = a->k.data; f.v = a->v.data;
    f.lg = a->log_gamma.data; f.la = a->log_alpha.data; f.g = a->g.data;
    f.mix = a->mix.data; f.gs = a->gla_scale.data;
    f.q_sb = a->q.stride[0]; f.q_sh = a->q.stride[1]; f.q_st = a->q.stride[2];
    f.k_sb = a->k.stride[0]; f.k_sh = a->k.stride[1]; f.k_st = a->k.stride[2];
    f.v_sb = a->v.stride[0]; f.v_sh = a->v.stride[1]; f.v_st = a->v.stride[2];
    f.lg_sb = a->log_gamma.stride[0]; f.lg_sh = a->log_gamma.stride[1]; f.lg_st = a->log_gamma.stride[2];
    f.la_sh = a->log_alpha.stride[0]; f.la_sj = a->log_alpha.stride[1];
    f.g_sb = a->g.stride[0]; f.g_sh = a->g.stride[1]; f.g_st = a->g.stride[2]; f.g_sj = a->g.stride[3];
    f.m_sb = a->mix.stride[0]; f.m_sh = a->mix.stride[1]; f.m_st = a->mix.stride[2];
    f.gs_sh = a->gla_scale.stride[0]; f.gs_sd = a->gla_scale.stride[1];
    f.lg_dt = a->log_gamma.dtype; f.la_dt = a->log_alpha.dtype; f.mix_dt = a->mix.dtype; f.gs_dt = a->gla_scale.dtype;
    f.B = a->B; f.H = a->H; f.T = a->T; f.R = a->R;
    f.nc = (a->T + C - 1) / C;
    k.dy = a->dy.data; k.n = a->n.data; k.o = a->o.data;
    k.rstd = a->rstd;
    k.s_in = (const uint16_t *)a->chunk_states;
    k.dq = (void *)a->dq.data; k.dk = (void *)a->dk.data; k.dv = (void *)a->dv.data;
    k.dlg = (void *)a->d_log_gamma.data; k.dg = (void *)a->d_g.data; k.dla = (void *)a->d_log_alpha.data;
    k.dmix = (void *)a->d_mix.data; k.dgs = (void *)a->d_gla_scale.data; k.dout = (void *)a->dout_attn.data;
    k.delta = a->delta;
    k.dy_sb = a->dy.stride[0]; k.dy_sh = a->dy.stride[1]; k.dy_st = a->dy.stride[2];
    k.n_sb = a->n.stride[0]; k.n_sh = a->n.stride[1]; k.n_st = a->n.stride[2];
    k.o_sb = a->o.stride[0]; k.o_sh = a->o.stride[1]; k.o_st = a->o.stride[2];
    k.dq_sb = a->dq.stride[0]; k.dq_sh = a->dq.stride[1]; k.dq_st = a->dq.stride[2];
    k.dk_sb = a->dk.stride[0]; k.dk_sh = a->dk.stride[1]; k.dk_st = a->dk.stride[2];
    k.dv_sb = a->dv.stride[0]; k.dv_sh = a->dv.stride[1]; k.dv_st = a->dv.stride[2];
    k.dlg_sb = a->d_log_gamma.stride[0]; k.dlg_sh = a->d_log_gamma.stride[1]; k.dlg_st = a->d_log_gamma.stride[2];
    k.dg_sb = a->d_g.stride[0]; k.dg_sh = a->d_g.stride[1]; k.dg_st = a->d_g.stride[2]; k.dg_sj = a->d_g.stride[3];
    k.dla_sh = a->d_log_alpha.stride[0]; k.dla_sj = a->d_log_alpha.stride[1];
    k.dmix_sb = a->d_mix.stride[0]; k.dmix_sh = a->d_mix.stride[1]; k.dmix_st = a->d_mix.stride[2];
    k.dgs_sh = a->d_gla_scale.stride[0]; k.dgs_sd = a->d_gla_scale.stride[1];
    k.do_sb = a->dout_attn.stride[0]; k.do_sh = a->dout_attn.stride[1]; k.do_st = a->dout_attn.stride[2];
    k.dlg_dt = a->d_log_gamma.dtype; k.dla_dt = a->d_log_alpha.dtype; k.dmix_dt = a->d_mix.dtype;
    k.dgs_dt = a->d_gla_scale.dtype;
    char *w = (char *)workspace;
    k.ws_do = w + L.dO;
    k.ws_dh = (float *)(w + L.dh);
    k.ws_gl = (float *)(w + L.gl);
    k.ds_end = (uint16_t *)(w + L.dse);
    k.dlg_part = (float *)(w + L.dlg);
    k.chunk_part = (float *)(w + L.cp);
    k.dgs_part = (float *)(w + L.dgs);
    k.part_la = (float *)(w + L.pla);
    k.part_gs = (float *)(w + L.pgs);
    f.unsafe = (uint8_t *)(w + L.flags);
    k.ntile = (a->T + ET - 1) / ET;
    const int J = a->D - a->R;
    hipStream_t s = (hipStream_t)stream;
    const bool gen = a->g.data != nullptr;
    switch (a->q.dtype) {
        case HOFA_F32: rc = gen ? dispatch<HOFA_F32, true>(k, a->D, J, s) : dispatch<HOFA_F32, false>(k, a->D, J, s); break;
        case HOFA_BF16: rc = gen ? dispatch<HOFA_BF16, true>(k, a->D, J, s) : dispatch<HOFA_BF16, false>(k, a->D, J, s); break;
        default: rc = gen ? dispatch<HOFA_F16, true>(k, a->D, J, s) : dispatch<HOFA_F16, false>(k, a->D, J, s); break;
    }
    if (rc) {
        set_error("hofa_gla_bwd: no kernel for this (D, J)");
        return rc;
    }
    return check_launch("hofa_gla_bwd");
}

// C ABI of the DSALT library: argument validation, workspace sizing and
// dispatch to the selection / forward / backward launchers.
#include <stdarg.h>
#include <stdio.h>

#include <map>
#include <mutex>
#include <string>

#include "attn.h"
#include "ce.h"
#include "ffn.h"
#include "probs.h"
#include "rope.h"
#include "select.h"
#include "common.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return DSALT_OK;
    return fail(DSALT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

size_t esize(int dtype) { return dtype == DSALT_DTYPE_F32 ? 4 : 2; }

int n_sets_of(const dsalt_problem& p) {
    if (p.select_mode == DSALT_SELECT_GLOBAL) return 1;
    return (p.max_seqlen + p.block_size - 1) / p.block_size;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

int check_problem(const dsalt_problem& p, bool attention) {
    if (p.total_len < 0 || p.num_seqs < 1) return fail(DSALT_ERR_INVALID, "total_len must be >= 0 and num_seqs >= 1");
    if (p.max_seqlen < 1 || (int64_t)p.max_seqlen > (int64_t)p.total_len + (p.total_len == 0))
        return fail(DSALT_ERR_INVALID, "max_seqlen %d outside [1, total_len=%d]", p.max_seqlen, p.total_len);
    if (p.n_heads < 1 || p.n_kv_heads < 1 || p.n_heads % p.n_kv_heads)
        return fail(DSALT_ERR_INVALID, "n_heads (%d) must be a positive multiple of n_kv_heads (%d)", p.n_heads,
                    p.n_kv_heads);
    if (attention) {
        if (p.head_dim != 64 && p.head_dim != 128)
            return fail(DSALT_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", p.head_dim);
    } else if (p.head_dim < 1 || (p.head_dim * esize(p.dtype)) % 16 || p.head_dim * esize(p.dtype) > 1024) {
        return fail(DSALT_ERR_INVALID, "head_dim %d must be a multiple of 16 bytes, at most 1024 bytes",
                    p.head_dim);
    }
    if (p.k_lmk < 0 || p.k_lmk > dsalt::kMaxLandmarks)
        return fail(DSALT_ERR_INVALID, "k_lmk %d outside [0, %d]", p.k_lmk, dsalt::kMaxLandmarks);
    if (p.select_mode != DSALT_SELECT_GLOBAL && p.select_mode != DSALT_SELECT_BLOCK)
        return fail(DSALT_ERR_INVALID, "unknown select_mode %d", p.select_mode);
    if (p.select_mode == DSALT_SELECT_BLOCK && p.block_size < 1)
        return fail(DSALT_ERR_INVALID, "block_size %d must be positive", p.block_size);
    if (p.dtype != DSALT_DTYPE_F32 && p.dtype != DSALT_DTYPE_BF16 && p.dtype != DSALT_DTYPE_F16)
        return fail(DSALT_ERR_INVALID, "unknown dtype %d", p.dtype);
    return DSALT_OK;
}

int check_rows(const void* ptr, int64_t st, int64_t sh, int dtype, const char* name) {
    if (!ptr) return fail(DSALT_ERR_INVALID, "%s is null", name);
    if (!aligned16(ptr)) return fail(DSALT_ERR_INVALID, "%s must be 16-byte aligned", name);
    size_t es = esize(dtype);
    if ((st * (int64_t)es) % 16 || (sh * (int64_t)es) % 16 || st <= 0 || sh < 0)
        return fail(DSALT_ERR_INVALID, "%s strides (%lld, %lld) must be positive multiples of 16 bytes", name,
                    (long long)st, (long long)sh);
    // runs of up to 1024 rows are addressed with 32-bit byte offsets from their first row
    if (st * (int64_t)es > (int64_t)(1u << 20))
        return fail(DSALT_ERR_UNSUPPORTED, "%s token stride of %lld bytes exceeds 1 MiB", name,
                    (long long)(st * (int64_t)es));
    return DSALT_OK;
}

dsalt::SelectParams select_params(const dsalt_select_args* a) {
    dsalt::SelectParams p = {};
    const dsalt_problem& q = a->p;
    p.total_len = q.total_len;
    p.num_seqs = q.num_seqs;
    p.max_seqlen = q.max_seqlen;
    p.n_heads = q.n_heads;
    p.n_kv_heads = q.n_kv_heads;
    p.head_dim = q.head_dim;
    p.k_lmk = q.k_lmk;
    p.select_mode = q.select_mode;
    p.block_size = q.block_size;
    p.dtype = q.dtype;
    p.hidden = a->hidden;
    p.stats_scope = a->stats_scope;
    p.n_sets = n_sets_of(q);
    p.h = a->h;
    p.h_stride_t = a->h_stride_t;
    p.v = a->v;
    p.v_stride_t = a->v_stride_t;
    p.v_stride_h = a->v_stride_h;
    p.alpha = a->alpha;
    p.w = a->w;
    p.cu = a->cu_seqlens;
    p.lmk_idx = a->lmk_idx;
    p.z_x = a->z_x;
    p.z_v = a->z_v;
    p.scores = a->scores;
    p.n_tiles = (q.max_seqlen + 63) / 64;
    if (a->plan) {  // the forward's row plan, carved as dsalt_fwd reads it
        dsalt::AttnParams ap = {};
        ap.num_seqs = q.num_seqs;
        ap.n_tiles = p.n_tiles;
        char* w = (char*)a->plan;
        dsalt::plan_carve(ap, w);
        p.plan_perm = ap.plan_perm;
        p.plan_bounds = ap.plan_bounds;
        p.tile_wmax = ap.tile_wmax;
    }
    return p;
}

int check_select(const dsalt_select_args* a) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    int rc = check_problem(a->p, false);
    if (rc) return rc;
    size_t es = esize(a->p.dtype);
    if (a->hidden <= 0 || (a->hidden * es) % 16)
        return fail(DSALT_ERR_INVALID, "hidden %d must be a positive multiple of 16 bytes", a->hidden);
    if (a->stats_scope != DSALT_STATS_PACKED && a->stats_scope != DSALT_STATS_SEQUENCE)
        return fail(DSALT_ERR_INVALID, "unknown stats_scope %d", a->stats_scope);
    if ((rc = check_rows(a->h, a->h_stride_t, 0, a->p.dtype, "h"))) return rc;
    if ((rc = check_rows(a->v, a->v_stride_t, a->v_stride_h, a->p.dtype, "v"))) return rc;
    if (!a->alpha || !a->w || !a->cu_seqlens || (a->p.k_lmk > 0 && !a->lmk_idx))
        return fail(DSALT_ERR_INVALID, "alpha, w, cu_seqlens and lmk_idx are required");
    if (a->p.select_mode == DSALT_SELECT_BLOCK && (a->z_x || a->z_v || a->scores))
        return fail(DSALT_ERR_INVALID, "z_x / z_v / scores are outputs of the global variant only");
    return DSALT_OK;
}

dsalt::AttnParams attn_common(const dsalt_problem& q, float scale) {
    dsalt::AttnParams p = {};
    p.total_len = q.total_len;
    p.num_seqs = q.num_seqs;
    p.max_seqlen = q.max_seqlen;
    p.n_heads = q.n_heads;
    p.n_kv_heads = q.n_kv_heads;
    p.head_dim = q.head_dim;
    p.k_lmk = q.k_lmk;
    p.n_sets = n_sets_of(q);
    p.block_size = q.select_mode == DSALT_SELECT_BLOCK ? q.block_size : 0;
    p.dtype = q.dtype;
    p.n_tiles = (q.max_seqlen + 63) / 64;
    p.scale = scale;
    p.c2 = scale * 1.4426950408889634f;
    p.inv_scale = 1.0f / scale;
    p.thr = 8.0f / p.c2;
    return p;
}

}  // namespace

extern "C" {

int dsalt_abi_version(void) { return DSALT_ABI_VERSION; }

const char* dsalt_last_error(void) { return g_err.c_str(); }

size_t dsalt_select_workspace_bytes(const dsalt_select_args* a) {
    if (check_select(a)) return 0;
    return dsalt::select_workspace(select_params(a));
}

size_t dsalt_select_workspace_bytes_cap(const dsalt_select_args* a, int border_cap) {
    if (check_select(a) || border_cap < 1) return 0;
    return dsalt::select_workspace_cap(select_params(a), border_cap);
}

int dsalt_select_with_border_cap(const dsalt_select_args* a, dsalt_stream_t stream, int border_cap) {
    int rc = check_select(a);
    if (rc) return rc;
    if (border_cap < 1) return fail(DSALT_ERR_INVALID, "border_cap must be >= 1");
    dsalt::SelectParams p = select_params(a);
    size_t need = dsalt::select_workspace_cap(p, border_cap);
    if (!a->workspace || a->workspace_bytes < need)
        return fail(DSALT_ERR_WORKSPACE, "selection needs %zu workspace bytes, got %zu", need, a->workspace_bytes);
    return hip_status(dsalt::select_launch(p, a->workspace, (hipStream_t)stream, border_cap), "dsalt_select");
}

int dsalt_select(const dsalt_select_args* a, dsalt_stream_t stream) {
    return dsalt_select_with_border_cap(a, stream, 1 << 30);
}

// Most landmark sets the rows of one 64-row tile belong to (block-causal sets).
static int max_sets_per_tile(const dsalt_problem& p) {
    if (p.select_mode != DSALT_SELECT_BLOCK || p.block_size % 64 == 0) return 1;
    int m = 1;
    for (int r0 = 0; r0 < p.max_seqlen; r0 += 64) {
        const int last = (r0 + 63 < p.max_seqlen ? r0 + 63 : p.max_seqlen - 1) / p.block_size;
        const int n = last - r0 / p.block_size + 1;
        if (n > m) m = n;
    }
    return m;
}

// forward parameters; `need_w` is false for the training variant (windows from w_cont)
static int fwd_params(const dsalt_fwd_args* a, bool need_w, dsalt::AttnParams* out) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    int rc = check_problem(a->p, true);
    if (rc) return rc;
    // sets of more than kSetSlots landmarks: the inference operator only
    if (!need_w && a->p.k_lmk > dsalt::kSetSlots)
        return fail(DSALT_ERR_UNSUPPORTED, "the training variant takes at most %d landmarks (k_lmk %d)", dsalt::kSetSlots,
                    a->p.k_lmk);
    // block sizes that are not multiples of 64: a tile's sets are staged in LDS together
    const int tsets = max_sets_per_tile(a->p);
    if (tsets > 1 && tsets * a->p.k_lmk > dsalt::kMultiSetSlots)
        return fail(DSALT_ERR_UNSUPPORTED,
                    "block_size %d: 64-row tiles span %d landmark sets; %d sets x k_lmk %d exceeds %d slots",
                    a->p.block_size, tsets, tsets, a->p.k_lmk, dsalt::kMultiSetSlots);
    const int dt = a->p.dtype;
    if ((rc = check_rows(a->q, a->q_stride_t, a->q_stride_h, dt, "q"))) return rc;
    if ((rc = check_rows(a->k, a->k_stride_t, a->k_stride_h, dt, "k"))) return rc;
    if ((rc = check_rows(a->v, a->v_stride_t, a->v_stride_h, dt, "v"))) return rc;
    if ((rc = check_rows(a->out, a->o_stride_t, a->o_stride_h, dt, "out"))) return rc;
    if ((need_w && !a->w) || !a->cu_seqlens || !a->lse || (a->p.k_lmk > 0 && !a->lmk_idx))
        return fail(DSALT_ERR_INVALID, "w, cu_seqlens, lse and lmk_idx are required");
    if (!(a->scale > 0.f)) return fail(DSALT_ERR_INVALID, "scale must be positive");
    dsalt::AttnParams p = attn_common(a->p, a->scale);
    p.q = a->q;
    p.q_st = a->q_stride_t;
    p.q_sh = a->q_stride_h;
    p.k = a->k;
    p.k_st = a->k_stride_t;
    p.k_sh = a->k_stride_h;
    p.v = a->v;
    p.v_st = a->v_stride_t;
    p.v_sh = a->v_stride_h;
    p.o = a->out;
    p.o_st = a->o_stride_t;
    p.o_sh = a->o_stride_h;
    p.lse_out = a->lse;
    p.w = a->w;
    p.cu = a->cu_seqlens;
    p.lmk = a->lmk_idx;
    p.lbias = a->lmk_bias;
    if (a->variant & ~DSALT_VARIANT_MASK) return fail(DSALT_ERR_INVALID, "unknown variant bits 0x%x", a->variant);
    p.variant = a->variant;
    *out = p;
    return DSALT_OK;
}

// training variant: soft-edge parameters on top of the operator's
static int train_params(const float* w_cont, float tau_win, float win_edge, dsalt::AttnParams* p) {
    if (!w_cont) return fail(DSALT_ERR_INVALID, "w_cont is required");
    if (!(tau_win > 0.f)) return fail(DSALT_ERR_INVALID, "tau_win must be positive");
    if (!(win_edge >= 0.f) || win_edge > 65536.f) return fail(DSALT_ERR_INVALID, "win_edge must be in [0, 65536]");
    if (p->block_size != 0) return fail(DSALT_ERR_UNSUPPORTED, "the training variant takes global landmark sets");
    p->w_cont = w_cont;
    p->tau_inv = 1.0f / tau_win;
    p->edge = win_edge;
    p->edge_keys = (int)ceilf(win_edge);
    return DSALT_OK;
}

static size_t wint_bytes(const dsalt::AttnParams& p) { return ((size_t)p.total_len * sizeof(int) + 255) & ~(size_t)255; }

size_t dsalt_plan_bytes(const dsalt_problem* p) {
    if (!p || check_problem(*p, true)) return 0;
    return dsalt::plan_bytes(attn_common(*p, 1.0f));
}

// the forward's only workspace is the row plan, which a caller-given plan buffer replaces
size_t dsalt_fwd_workspace_bytes(const dsalt_fwd_args* a) {
    if (!a || check_problem(a->p, true)) return 0;
    return a->plan ? 0 : dsalt::plan_bytes(attn_common(a->p, 1.0f));
}

int dsalt_fwd(const dsalt_fwd_args* a, dsalt_stream_t stream) {
    dsalt::AttnParams p;
    int rc = fwd_params(a, true, &p);
    if (rc) return rc;
    const size_t need = a->plan ? 0 : dsalt::plan_bytes(p);
    if (need && (!a->workspace || a->workspace_bytes < need))
        return fail(DSALT_ERR_WORKSPACE, "forward needs %zu workspace bytes, got %zu", need, a->workspace_bytes);
    return hip_status(dsalt::fwd_launch(p, a->workspace, a->plan, a->plan_ready != 0, (hipStream_t)stream),
                      "dsalt_fwd");
}

}  // extern "C"

// ------------------------------------------------ forward without allocations
// The row plan of dsalt_fwd_noalloc lives in this file-scope device array (one copy per
// GPU, held until the process ends).  In host code `scratch` names a host-side stand-in,
// not a device address: the address is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address is used.
namespace {

constexpr size_t kScratchBytes = DSALT_FWD_NOALLOC_MAX_PLAN_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::map<int, void*> g_scratch_ptr;  // device -> address of its copy of `scratch`

// address of `scratch` on device `dev` (looked up on the first call for that device)
hipError_t scratch_on(int dev, void** out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_ptr.find(dev);
    if (it != g_scratch_ptr.end()) {
        *out = it->second;
        return hipSuccess;
    }
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) {
        const hipError_t e2 = hipSetDevice(cur);
        if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess) return e;
    if (ptr == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = ptr;
    *out = ptr;
    return hipSuccess;
}

}  // namespace

extern "C" {

int dsalt_fwd_noalloc(const dsalt_fwd_args* a, dsalt_stream_t stream) {
    dsalt::AttnParams p;
    int rc = fwd_params(a, true, &p);
    if (rc) return rc;
    const size_t need = dsalt::plan_bytes(p);
    if (!a->plan && need > kScratchBytes)
        return fail(DSALT_ERR_WORKSPACE,
                    "dsalt_fwd_noalloc: the row plan needs %zu bytes, more than its %zu-byte device scratch "
                    "(use dsalt_fwd with a workspace)", need, kScratchBytes);
    void* ws = nullptr;
    if (!a->plan) {
        int dev = -1;
        hipError_t e = stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev);
        if (e == hipSuccess) e = scratch_on(dev, &ws);
        if (e != hipSuccess) return hip_status(e, "dsalt_fwd_noalloc scratch");
    }
    // every kernel writes each plan entry it later reads: nothing needs clearing
    return hip_status(dsalt::fwd_launch(p, ws, a->plan, a->plan_ready != 0, (hipStream_t)stream),
                      "dsalt_fwd_noalloc");
}

size_t dsalt_train_fwd_workspace_bytes(const dsalt_train_fwd_args* a) {
    if (!a || check_problem(a->base.p, true)) return 0;
    const dsalt::AttnParams p = attn_common(a->base.p, 1.0f);
    return wint_bytes(p) + (a->base.plan ? 0 : dsalt::plan_bytes(p));
}

int dsalt_train_fwd(const dsalt_train_fwd_args* a, dsalt_stream_t stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    dsalt::AttnParams p;
    int rc = fwd_params(&a->base, false, &p);
    if (rc) return rc;
    if ((rc = train_params(a->w_cont, a->tau_win, a->win_edge, &p))) return rc;
    const size_t need = wint_bytes(p) + (a->base.plan ? 0 : dsalt::plan_bytes(p));
    if (!a->base.workspace || a->base.workspace_bytes < need)
        return fail(DSALT_ERR_WORKSPACE, "training forward needs %zu workspace bytes, got %zu", need,
                    a->base.workspace_bytes);
    int* w_int = (int*)a->base.workspace;
    p.w = w_int;
    hipError_t e = dsalt::train_windows_launch(p, w_int, (hipStream_t)stream);
    if (e == hipSuccess)
        e = dsalt::fwd_launch(p, (char*)a->base.workspace + wint_bytes(p), a->base.plan, false, (hipStream_t)stream);
    return hip_status(e, "dsalt_train_fwd");
}

static int bwd_params(const dsalt_bwd_args* a, dsalt::AttnParams* out, bool need_w = true) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    int rc = check_problem(a->p, true);
    if (rc) return rc;
    if (!need_w && a->p.k_lmk > dsalt::kSetSlots)
        return fail(DSALT_ERR_UNSUPPORTED, "the training variant takes at most %d landmarks (k_lmk %d)", dsalt::kSetSlots,
                    a->p.k_lmk);
    if (a->p.select_mode != DSALT_SELECT_GLOBAL)
        return fail(DSALT_ERR_UNSUPPORTED, "backward of the block-causal variant is not implemented");
    const int dt = a->p.dtype;
    if ((rc = check_rows(a->q, a->q_stride_t, a->q_stride_h, dt, "q"))) return rc;
    if ((rc = check_rows(a->k, a->k_stride_t, a->k_stride_h, dt, "k"))) return rc;
    if ((rc = check_rows(a->v, a->v_stride_t, a->v_stride_h, dt, "v"))) return rc;
    if ((rc = check_rows(a->out, a->o_stride_t, a->o_stride_h, dt, "out"))) return rc;
    if ((rc = check_rows(a->dout, a->do_stride_t, a->do_stride_h, dt, "dout"))) return rc;
    if (!a->dq || !a->dk || !a->dv || !aligned16(a->dq) || !aligned16(a->dk) || !aligned16(a->dv))
        return fail(DSALT_ERR_INVALID, "dq, dk, dv must be non-null and 16-byte aligned");
    if ((need_w && !a->w) || !a->cu_seqlens || !a->lse || (a->p.k_lmk > 0 && !a->lmk_idx))
        return fail(DSALT_ERR_INVALID, "w, cu_seqlens, lse and lmk_idx are required");
    if (!(a->scale > 0.f)) return fail(DSALT_ERR_INVALID, "scale must be positive");
    dsalt::AttnParams p = attn_common(a->p, a->scale);
    p.q = a->q;
    p.q_st = a->q_stride_t;
    p.q_sh = a->q_stride_h;
    p.k = a->k;
    p.k_st = a->k_stride_t;
    p.k_sh = a->k_stride_h;
    p.v = a->v;
    p.v_st = a->v_stride_t;
    p.v_sh = a->v_stride_h;
    p.o = a->out;
    p.o_st = a->o_stride_t;
    p.o_sh = a->o_stride_h;
    p.dout = a->dout;
    p.do_st = a->do_stride_t;
    p.do_sh = a->do_stride_h;
    p.lse = a->lse;
    p.w = a->w;
    p.cu = a->cu_seqlens;
    p.lmk = a->lmk_idx;
    p.lbias = a->lmk_bias;
    p.dq = a->dq;
    p.dk = a->dk;
    p.dv = a->dv;
    p.d_bias = a->d_bias;
    if (a->variant & ~DSALT_VARIANT_MASK) return fail(DSALT_ERR_INVALID, "unknown variant bits 0x%x", a->variant);
    p.variant = a->variant;
    *out = p;
    return DSALT_OK;
}

size_t dsalt_bwd_workspace_bytes(const dsalt_bwd_args* a) {
    dsalt::AttnParams p;
    if (bwd_params(a, &p)) return 0;
    return dsalt::bwd_workspace(p, a->plan != nullptr);
}

int dsalt_bwd(const dsalt_bwd_args* a, dsalt_stream_t stream) {
    dsalt::AttnParams p;
    int rc = bwd_params(a, &p);
    if (rc) return rc;
    size_t need = dsalt::bwd_workspace(p, a->plan != nullptr);
    if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
        return fail(DSALT_ERR_WORKSPACE, "backward needs %zu workspace bytes, got %zu", need, a->workspace_bytes);
    return hip_status(dsalt::bwd_launch(p, a->workspace, a->plan, (hipStream_t)stream), "dsalt_bwd");
}

// training backward workspace: integer windows, per-head d w~, then the operator's
static size_t train_bwd_extra(const dsalt::AttnParams& p) {
    return wint_bytes(p) + (((size_t)p.total_len * p.n_heads * sizeof(float) + 255) & ~(size_t)255);
}

size_t dsalt_train_bwd_workspace_bytes(const dsalt_train_bwd_args* a) {
    dsalt::AttnParams p;
    if (!a || bwd_params(&a->base, &p, false)) return 0;
    return train_bwd_extra(p) + dsalt::bwd_workspace(p, a->base.plan != nullptr);
}

int dsalt_train_bwd(const dsalt_train_bwd_args* a, dsalt_stream_t stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    dsalt::AttnParams p;
    int rc = bwd_params(&a->base, &p, false);
    if (rc) return rc;
    if ((rc = train_params(a->w_cont, a->tau_win, a->win_edge, &p))) return rc;
    if (!a->d_w) return fail(DSALT_ERR_INVALID, "d_w is required");
    const size_t need = train_bwd_extra(p) + dsalt::bwd_workspace(p, a->base.plan != nullptr);
    if (!a->base.workspace || a->base.workspace_bytes < need || !aligned16(a->base.workspace))
        return fail(DSALT_ERR_WORKSPACE, "training backward needs %zu workspace bytes, got %zu", need,
                    a->base.workspace_bytes);
    char* w = (char*)a->base.workspace;
    int* w_int = (int*)w;
    p.w = w_int;
    p.dw_h = (float*)(w + wint_bytes(p));
    p.d_w = a->d_w;
    hipError_t e = dsalt::train_windows_launch(p, w_int, (hipStream_t)stream);
    if (e == hipSuccess) e = dsalt::bwd_launch(p, w + train_bwd_extra(p), a->base.plan, (hipStream_t)stream);
    if (e == hipSuccess) e = dsalt::train_dw_launch(p, (hipStream_t)stream);
    return hip_status(e, "dsalt_train_bwd");
}

int dsalt_rope_qk(const dsalt_rope_args* a, dsalt_stream_t stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    if (a->total_len < 0 || a->num_seqs < 1 || a->n_q_heads < 0 || a->n_k_heads < 0)
        return fail(DSALT_ERR_INVALID, "bad shape (T=%d, S=%d, heads %d/%d)", a->total_len, a->num_seqs,
                    a->n_q_heads, a->n_k_heads);
    if (a->head_dim < 16 || a->head_dim > 256 || a->head_dim % 16)
        return fail(DSALT_ERR_INVALID, "head_dim must be a multiple of 16 in [16, 256], got %d", a->head_dim);
    if (a->dtype < 0 || a->dtype > 2) return fail(DSALT_ERR_INVALID, "unknown dtype %d", a->dtype);
    if (a->max_seqlen < 0 || a->max_seqlen > a->max_pos)
        return fail(DSALT_ERR_INVALID, "max_seqlen (%d) must be in [0, max_pos = %d]", a->max_seqlen, a->max_pos);
    int rc;
    if (a->n_q_heads && (rc = check_rows(a->q, a->q_stride_t, a->q_stride_h, a->dtype, "q"))) return rc;
    if (a->n_k_heads && (rc = check_rows(a->k, a->k_stride_t, a->k_stride_h, a->dtype, "k"))) return rc;
    if (!a->cu_seqlens || !a->cos || !a->sin || !aligned16(a->cos) || !aligned16(a->sin))
        return fail(DSALT_ERR_INVALID, "cu_seqlens, cos and sin are required (cos/sin 16-byte aligned)");
    dsalt::RopeParams p;
    p.total_len = a->total_len;
    p.num_seqs = a->num_seqs;
    p.n_q_heads = a->n_q_heads;
    p.n_k_heads = a->n_k_heads;
    p.head_dim = a->head_dim;
    p.dtype = a->dtype;
    p.q = a->q;
    p.q_st = a->q_stride_t;
    p.q_sh = a->q_stride_h;
    p.k = a->k;
    p.k_st = a->k_stride_t;
    p.k_sh = a->k_stride_h;
    p.cu = a->cu_seqlens;
    p.cos = a->cos;
    p.sin = a->sin;
    p.max_pos = a->max_pos;
    return hip_status(dsalt::rope_launch(p, (hipStream_t)stream), "dsalt_rope_qk");
}

int dsalt_export_probs(const dsalt_probs_args* a, dsalt_stream_t stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    int rc = check_problem(a->p, true);
    if (rc) return rc;
    const int dt = a->p.dtype;
    if ((rc = check_rows(a->q, a->q_stride_t, a->q_stride_h, dt, "q"))) return rc;
    if ((rc = check_rows(a->k, a->k_stride_t, a->k_stride_h, dt, "k"))) return rc;
    if (!a->w || !a->cu_seqlens || !a->lse || (a->p.k_lmk > 0 && !a->lmk_idx))
        return fail(DSALT_ERR_INVALID, "w, cu_seqlens, lse and lmk_idx are required");
    if (a->seq < 0 || a->seq >= a->p.num_seqs) return fail(DSALT_ERR_INVALID, "seq %d out of range", a->seq);
    if (a->rows < 0 || a->rows > a->p.max_seqlen || a->w_cap < 1)
        return fail(DSALT_ERR_INVALID, "rows must be in [0, max_seqlen] and w_cap >= 1");
    if (!a->p_win) return fail(DSALT_ERR_INVALID, "p_win is required");
    if (!(a->scale > 0.f)) return fail(DSALT_ERR_INVALID, "scale must be positive");
    dsalt::ProbsParams pp;
    pp.a = attn_common(a->p, a->scale);
    pp.a.q = a->q;
    pp.a.q_st = a->q_stride_t;
    pp.a.q_sh = a->q_stride_h;
    pp.a.k = a->k;
    pp.a.k_st = a->k_stride_t;
    pp.a.k_sh = a->k_stride_h;
    pp.a.w = a->w;
    pp.a.cu = a->cu_seqlens;
    pp.a.lmk = a->lmk_idx;
    pp.a.lbias = a->lmk_bias;
    pp.a.lse_out = (float*)a->lse;
    pp.seq = a->seq;
    pp.out_rows = a->rows;
    pp.w_cap = a->w_cap;
    pp.p_win = a->p_win;
    pp.p_lmk = a->p.k_lmk > 0 ? a->p_lmk : nullptr;
    return hip_status(dsalt::probs_launch(pp, (hipStream_t)stream), "dsalt_export_probs");
}

int dsalt_cross_entropy_rows(const dsalt_ce_args* a, dsalt_stream_t stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    if (a->rows < 0 || a->n_cols < 1)
        return fail(DSALT_ERR_INVALID, "rows >= 0 and n_cols >= 1 required (got %d, %d)", a->rows, a->n_cols);
    if (a->dtype < 0 || a->dtype > 2) return fail(DSALT_ERR_INVALID, "unknown dtype %d", a->dtype);
    if (a->reduction < 0 || a->reduction > 2) return fail(DSALT_ERR_INVALID, "reduction must be 0, 1 or 2");
    if (a->rows == 0) return DSALT_OK;
    if (!a->logits || !aligned16(a->logits) || a->logits_stride < a->n_cols ||
        (a->logits_stride * (int64_t)esize(a->dtype)) % 16)
        return fail(DSALT_ERR_INVALID, "logits need 16-byte aligned rows of at least n_cols elements");
    if (!a->target || !a->loss) return fail(DSALT_ERR_INVALID, "target and loss are required");
    if (!(a->label_smoothing >= 0.f && a->label_smoothing <= 1.f))
        return fail(DSALT_ERR_INVALID, "label_smoothing must be in [0, 1]");
    if (!(a->softcap >= 0.f)) return fail(DSALT_ERR_INVALID, "softcap must be >= 0 (0: none)");
    dsalt::CeParams p;
    p.rows = a->rows;
    p.n_cols = a->n_cols;
    p.dtype = a->dtype;
    p.x = a->logits;
    p.x_st = a->logits_stride;
    p.target = a->target;
    p.ce_weight = a->ce_weight;
    p.loss = a->loss;
    p.z_loss = a->z_loss;
    p.accuracy = a->accuracy;
    p.predicted = a->predicted;
    p.ignore_index = a->ignore_index;
    p.n_non_ignore = a->n_non_ignore;
    p.sum_non_ignore_weight = a->sum_non_ignore_weight;
    p.weight_sum = a->weight_sum;
    p.lse_square_scale = a->lse_square_scale;
    p.label_smoothing = a->label_smoothing;
    p.softcap = a->softcap;
    p.reduction = a->reduction;
    p.grads = a->want_grad;
    p.token_scaling = a->token_scaling;
    return hip_status(dsalt::ce_launch(p, (hipStream_t)stream), "dsalt_cross_entropy_rows");
}

int dsalt_silu_mul(const dsalt_silu_mul_args* a, dsalt_stream_t stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    if (a->rows < 0 || a->cols < 0)
        return fail(DSALT_ERR_INVALID, "rows >= 0 and cols >= 0 required (got %d x %d)", a->rows, a->cols);
    if (a->dtype < 0 || a->dtype > 2) return fail(DSALT_ERR_INVALID, "unknown dtype %d", a->dtype);
    if (a->rows == 0 || a->cols == 0) return DSALT_OK;
    const int64_t es = (int64_t)esize(a->dtype);
    const void* ptrs[3] = {a->gate, a->up, a->out};
    const int64_t strides[3] = {a->gate_stride, a->up_stride, a->out_stride};
    for (int i = 0; i < 3; ++i)
        if (!ptrs[i] || !aligned16(ptrs[i]) || strides[i] < a->cols || (strides[i] * es) % 16)
            return fail(DSALT_ERR_INVALID, "gate, up and out need 16-byte aligned rows of at least cols elements");
    dsalt::SiluMulParams p;
    p.rows = a->rows;
    p.cols = a->cols;
    p.dtype = a->dtype;
    p.gate = a->gate;
    p.gate_st = a->gate_stride;
    p.up = a->up;
    p.up_st = a->up_stride;
    p.out = a->out;
    p.out_st = a->out_stride;
    return hip_status(dsalt::silu_mul_launch(p, (hipStream_t)stream), "dsalt_silu_mul");
}

int dsalt_gather_landmarks(const dsalt_gather_args* a, dsalt_stream_t stream) {
    if (!a) return fail(DSALT_ERR_INVALID, "null argument struct");
    int rc = check_problem(a->p, false);
    if (rc) return rc;
    const int dt = a->p.dtype;
    if ((rc = check_rows(a->k, a->k_stride_t, a->k_stride_h, dt, "k"))) return rc;
    if ((rc = check_rows(a->v, a->v_stride_t, a->v_stride_h, dt, "v"))) return rc;
    if (!a->cu_seqlens || !a->lmk_idx || !a->lmk_k || !a->lmk_v || !aligned16(a->lmk_k) || !aligned16(a->lmk_v))
        return fail(DSALT_ERR_INVALID, "cu_seqlens, lmk_idx, lmk_k, lmk_v are required (16-byte aligned)");
    dsalt::GatherParams p;
    p.total_len = a->p.total_len;
    p.num_seqs = a->p.num_seqs;
    p.max_seqlen = a->p.max_seqlen;
    p.n_heads = a->p.n_heads;
    p.n_kv_heads = a->p.n_kv_heads;
    p.head_dim = a->p.head_dim;
    p.k_lmk = a->p.k_lmk;
    p.n_sets = n_sets_of(a->p);
    p.dtype = dt;
    p.k = a->k;
    p.k_stride_t = a->k_stride_t;
    p.k_stride_h = a->k_stride_h;
    p.v = a->v;
    p.v_stride_t = a->v_stride_t;
    p.v_stride_h = a->v_stride_h;
    p.cu = a->cu_seqlens;
    p.lmk_idx = a->lmk_idx;
    p.lmk_k = a->lmk_k;
    p.lmk_v = a->lmk_v;
    return hip_status(dsalt::gather_launch(p, (hipStream_t)stream), "dsalt_gather_landmarks");
}

}  // extern "C"

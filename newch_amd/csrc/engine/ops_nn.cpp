// softmax / log_softmax over the last axis, LayerNorm over the last k axes, and the losses built on
// the softmax rows.  Reference: engine/src/ops/ops_nn.c (:8-77 softmax, :83-162 cross_entropy and
// mse_loss, :368-426 nll_loss, :434-538 layer_norm).
#include "engine.hpp"

namespace nce {

enum { SM_LOG = 0, SM_PLAIN = 1 };

// softmax rows are the last axis
static nc_status softmax_shape(nc_node *n, OutSpec &out) {
    if (!inputs_f32(n, 0, 1)) return NC_ERR_DTYPE;
    out.dims = Dims::of(n->in[0]);
    if (out.dims.rank == 0) return reject(n, NC_ERR_SHAPE, "%s: input must have at least 1 dimension", n->op->name);
    return NC_OK;
}

static void rows_cols(const nc_tensor *t, int64_t *rows, int64_t *C) {
    *C = t->shape[t->ndim - 1];
    *rows = *C ? nc_numel(t) / *C : 0;
}

static nc_status softmax_fwd(nc_node *n) {
    nc_ctx *ctx = n->out->ctx;
    float *x = contig_f32(n->in[0]), *y = fptr(n->out);
    if (!x || !y) return NC_ERR_STATE;
    int64_t rows, C;
    rows_cols(n->out, &rows, &C);
    if (!hip_layer_ok(ctx, nc_hip_softmax_fwd(n->op->kind == SM_LOG, rows, C, x, y, stream(ctx)), n->op->name))
        return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

static void softmax_bwd(nc_node *n) {
    nc_tensor *in = n->in[0];
    nc_ctx *ctx = in->ctx;
    if (!grad_buf(in)) return;
    float *y = fptr(n->out), *g = fptr(n->out->grad);
    if (!y || !g) return;
    const int acc = grad_acc(in);
    float *gi = fptr(in->grad);
    if (!gi) return;
    int64_t rows, C;
    rows_cols(n->out, &rows, &C);
    if (!hip_layer_ok(ctx, nc_hip_softmax_bwd(n->op->kind == SM_LOG, rows, C, y, g, gi, acc, stream(ctx)),
                      n->op->name))
        return;
    wrote_dev(in->grad);
}

const OpDef op_log_softmax = {"log_softmax", 0, SM_LOG, softmax_shape, nullptr, softmax_fwd, softmax_bwd};
const OpDef op_softmax = {"softmax", 0, SM_PLAIN, softmax_shape, nullptr, softmax_fwd, softmax_bwd};

// ---- layer norm ------------------------------------------------------------------------------------
// inputs: x, then weight and bias when present (p.i[1], p.i[2]).  The rows are x's last k axes
// flattened (k = p.i[0]); weight and bias hold one value per row element.
static nc_status layer_norm_shape(nc_node *n, OutSpec &out) {
    if (!inputs_f32(n, 0, n->n_in)) return NC_ERR_DTYPE;
    out.dims = Dims::of(n->in[0]);
    const int k = (int)n->p.i[0];
    if (k < 1 || k > out.dims.rank)
        return reject(n, NC_ERR_SHAPE, "layer_norm: normalized_shape has %d dims, input only %d", k, out.dims.rank);
    int64_t row = 1;
    for (int j = 0; j < k; j++) row *= out.dims.back(j);
    for (int i = 1; i < n->n_in; i++)
        if (nc_numel(n->in[i]) != row)
            return reject(n, NC_ERR_SHAPE, "layer_norm: weight/bias need %lld elements, got %lld", (long long)row,
                          (long long)nc_numel(n->in[i]));
    return NC_OK;
}

static int64_t ln_dim(const nc_node *n) {
    const nc_tensor *x = n->in[0];
    const int k = (int)n->p.i[0];
    return shape_numel(k, x->shape + x->ndim - k);
}

static nc_status layer_norm_fwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    const int has_w = (int)n->p.i[1], has_b = (int)n->p.i[2];
    float *w = has_w ? contig_f32(n->in[1]) : nullptr;
    float *b = has_b ? contig_f32(n->in[1 + has_w]) : nullptr;
    float *X = contig_f32(x), *Y = fptr(n->out);
    const int64_t D = ln_dim(n), R = D ? nc_numel(x) / D : 0;
    // per-row {mean, rstd}, read again by the backward
    float *stats = (float *)save_state(n, (size_t)(2 * R + 1) * sizeof(float));
    if (!X || !Y || !stats || (has_w && !w) || (has_b && !b)) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_layer_norm_fwd(R, D, X, w, b, n->p.f[0], Y, stats, stream(ctx)), "layer_norm"))
        return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

static void layer_norm_bwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    const int has_w = (int)n->p.i[1], has_b = (int)n->p.i[2];
    nc_tensor *wt = has_w ? n->in[1] : nullptr, *bt = has_b ? n->in[1 + has_w] : nullptr;
    float *X = contig_f32(x), *w = wt ? contig_f32(wt) : nullptr, *g = fptr(n->out->grad);
    const int64_t D = ln_dim(n), R = D ? nc_numel(x) / D : 0;
    if (!X || (wt && !w) || !g) return;
    const bool want_x = needs_grad(x), want_w = wt && needs_grad(wt), want_b = bt && needs_grad(bt);
    if ((want_x && !grad_buf(x)) || (want_w && !grad_buf(wt)) || (want_b && !grad_buf(bt))) return;
    const int acc = want_x ? grad_acc(x) : 1;
    float *gx = want_x ? fptr(x->grad) : nullptr;
    // column sums are added into gw / gb: a fresh buffer is given its zeros by fptr
    float *gw = want_w ? fptr(wt->grad) : nullptr;
    float *gb = want_b ? fptr(bt->grad) : nullptr;
    if ((want_x && !gx) || (want_w && !gw) || (want_b && !gb)) return;
    const size_t ws_bytes = (want_w || want_b) ? nc_hip_layer_norm_bwd_workspace(R, D) : 0;
    char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
    if (ws_bytes && !ws) return;
    if (!hip_layer_ok(ctx,
                      nc_hip_layer_norm_bwd(R, D, X, w, (const float *)n->saved, g, gx, gw, gb, acc, ws, ws_bytes,
                                            stream(ctx)),
                      "layer_norm"))
        return;
    if (gx) wrote_dev(x->grad);
    if (gw) wrote_dev(wt->grad);
    if (gb) wrote_dev(bt->grad);
}

const OpDef op_layer_norm = {"layer_norm", 0, 0, layer_norm_shape, nullptr, layer_norm_fwd, layer_norm_bwd};

// ---- losses ----------------------------------------------------------------------------------------
// cross_entropy (ops_nn.c:83-156) and nll_loss (ops_nn.c:368-426): f32 rows [N, C], i32 labels [N],
// a 0-d f32 loss.  The forward keeps a copy of the labels for the backward, as the reference does,
// and for cross entropy each row's maximum and log-sum-exp (8 bytes per row, where the reference keeps
// the [N, C] probabilities: the backward recomputes them from the logits with the same fp32
// operations); it reads the kernel's label check back before returning so an out-of-range label
// fails the call the reference's way.
enum { LOSS_CE = 0, LOSS_NLL = 1 };

static nc_status loss_shape(nc_node *n, OutSpec &out) {
    const bool ce = n->op->kind == LOSS_CE;
    if (!inputs_f32(n, 0, 1)) return NC_ERR_DTYPE;
    if (n->in[1]->dtype != NC_I32) return reject(n, NC_ERR_DTYPE, "%s: labels must be i32", n->op->name);
    const Dims x = Dims::of(n->in[0]), y = Dims::of(n->in[1]);
    const bool rows_match = x.rank == 2 && y.rank == 1 && y.e[0] == x.e[0];
    if (!rows_match || (ce && x.e[1] < 1)) {
        char tx[96], ty[96];
        return reject(n, NC_ERR_SHAPE, "%s: expected %s [N, C] and labels [N], got %s and %s", n->op->name,
                      ce ? "logits" : "log-probabilities", x.text(tx, sizeof tx), y.text(ty, sizeof ty));
    }
    out.dims = Dims{};  // a 0-d loss
    return NC_OK;
}

// The loss forwards' bad-label key lands in a pinned host word the kernel writes directly (mapped
// into the device's address space), so the host reads it after the stream synchronisation the
// reference's synchronous error needs anyway, with no device-to-host copy.  Null when the host
// allocation is refused: the key then goes through arena memory and a copy.
static uint64_t *loss_flag_dev(nc_ctx *ctx) {
    if (!ctx->loss_flag) {
        void *h = nullptr, *d = nullptr;
        if (hipHostMalloc(&h, sizeof(uint64_t), hipHostMallocMapped | hipHostMallocPortable) != hipSuccess || !h) {
            (void)hipGetLastError();
            return nullptr;
        }
        if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || !d) {
            (void)hipGetLastError();
            (void)hipHostFree(h);
            return nullptr;
        }
        ctx->loss_flag = (uint64_t *)h;
        ctx->loss_flag_dev = (uint64_t *)d;
    }
    return ctx->loss_flag_dev;
}

static nc_status loss_fwd(nc_node *n) {
    nc_tensor *xt = n->in[0], *yt = n->in[1];
    nc_ctx *ctx = xt->ctx;
    const bool ce = n->op->kind == LOSS_CE;
    const int64_t N = xt->shape[0], C = xt->shape[1];
    float *x = contig_f32(xt), *loss = fptr(n->out);
    char *labels = dptr(yt);
    if (!x || !loss || !labels) return NC_ERR_STATE;
    // saved block: [row statistics N x {max, log-sum-exp} floats (cross entropy)][labels N int32]
    const size_t pbytes = ce ? (size_t)N * 2 * sizeof(float) : 0;
    const size_t sbytes = pbytes + (size_t)(N ? N : 1) * sizeof(int32_t);
    char *saved = (char *)save_state(n, sbytes);
    const size_t ws_bytes = nc_hip_loss_workspace(N, C);
    char *ws = arena_alloc(ctx, ws_bytes ? ws_bytes : 8);
    uint64_t *const mapped = loss_flag_dev(ctx);
    uint64_t *bad = mapped ? mapped : (uint64_t *)arena_alloc(ctx, sizeof(uint64_t));
    if (!saved || !ws || !bad) return NC_ERR_STATE;
    float *stats = ce ? (float *)saved : nullptr;
    int32_t *lab = (int32_t *)(saved + pbytes);
    if (N > 0 && !hip_layer_ok(ctx, nc_hip_copy_strided(4, 1, yt->shape, labels, yt->stride, lab, stream(ctx)),
                               n->op->name))
        return NC_ERR_STATE;
    const int rc = ce ? nc_hip_cross_entropy_fwd(N, C, x, lab, stats, loss, bad, ws, ws_bytes, stream(ctx))
                      : nc_hip_nll_loss_fwd(N, C, x, lab, (int)n->p.i[0], loss, bad, ws, ws_bytes, stream(ctx));
    if (!hip_layer_ok(ctx, rc, n->op->name)) return NC_ERR_STATE;
    uint64_t hb = 0;
    if (!mapped && !hip_ok(ctx, hipMemcpyAsync(&hb, bad, sizeof hb, hipMemcpyDeviceToHost, stream(ctx)), n->op->name))
        return NC_ERR_STATE;
    if (!hip_ok(ctx, hipStreamSynchronize(stream(ctx)), n->op->name)) return NC_ERR_STATE;
    if (mapped) hb = *(volatile const uint64_t *)ctx->loss_flag;
    if (hb != ~(uint64_t)0) {
        error(ctx, NC_ERR_ARG, "%s: label %d at row %lld outside [0, %lld)", n->op->name, (int32_t)(uint32_t)hb,
              (long long)(hb >> 32), (long long)C);
        return NC_ERR_ARG;
    }
    wrote_dev(n->out);
    // the backward recomputes the probabilities from these logits: it refuses logits written since
    n->p.i[1] = (int64_t)owner_of(xt)->wgen;
    return NC_OK;
}

static void loss_bwd(nc_node *n) {
    nc_tensor *xt = n->in[0];
    nc_ctx *ctx = xt->ctx;
    const bool ce = n->op->kind == LOSS_CE;
    const int64_t N = xt->shape[0], C = xt->shape[1];
    if (ce && owner_of(xt)->wgen != (uint64_t)n->p.i[1]) {
        error(ctx, NC_ERR_STATE,
              "cross_entropy: the logits were written after the forward (the backward recomputes the "
              "probabilities from them)");
        return;
    }
    if (!grad_buf(xt)) return;
    float *g = fptr(n->out->grad);
    if (!g) return;
    const char *saved = (const char *)n->saved;
    const size_t pbytes = ce ? (size_t)N * 2 * sizeof(float) : 0;
    const int32_t *lab = (const int32_t *)(saved + pbytes);
    int acc = grad_acc(xt);
    if (!ce && !acc) {  // only the labels' entries change: the rest of a fresh buffer needs its zeros
        if (!fill_zero(xt->grad)) return;
        acc = 1;
    }
    float *gi = fptr(xt->grad);
    const float *x = ce ? contig_f32(xt) : nullptr;  // the logits the probabilities are recomputed from
    if (!gi || (ce && !x)) return;
    const int rc = ce ? nc_hip_cross_entropy_bwd(N, C, x, (const float *)saved, lab, g, gi, acc, stream(ctx))
                      : nc_hip_nll_loss_bwd(N, C, lab, g, (int)n->p.i[0], gi, stream(ctx));
    if (!hip_layer_ok(ctx, rc, n->op->name)) return;
    wrote_dev(xt->grad);
}

const OpDef op_cross_entropy = {"cross_entropy", 0, LOSS_CE, loss_shape, nullptr, loss_fwd, loss_bwd};
const OpDef op_nll_loss = {"nll_loss", 0, LOSS_NLL, loss_shape, nullptr, loss_fwd, loss_bwd};

}  // namespace nce

using namespace nce;

extern "C" {
nc_tensor *nc_log_softmax(nc_tensor *x) { return apply(&op_log_softmax, &x, 1, nullptr); }
nc_tensor *nc_softmax(nc_tensor *x) { return apply(&op_softmax, &x, 1, nullptr); }

nc_tensor *nc_cross_entropy(nc_tensor *logits, nc_tensor *labels) {
    nc_tensor *in[2] = {logits, labels};
    return apply(&op_cross_entropy, in, 2, nullptr);
}

nc_tensor *nc_nll_loss(nc_tensor *logp, nc_tensor *labels, int sum) {
    nc_tensor *in[2] = {logp, labels};
    Params p{};
    p.i[0] = sum ? 1 : 0;
    return apply(&op_nll_loss, in, 2, &p);
}

// composite, differentiable through the ops it is built from (ops_nn.c:158-162)
nc_tensor *nc_mse_loss(nc_tensor *pred, nc_tensor *target) {
    nc_tensor *d = nc_sub(pred, target);
    return nc_mean(nc_mul(d, d), NC_ALL_AXES, 0);
}

nc_tensor *nc_layer_norm(nc_tensor *x, int normalized_ndim, nc_tensor *weight, nc_tensor *bias, float eps) {
    nc_tensor *in[3] = {x, nullptr, nullptr};
    int k = 1;
    if (weight) in[k++] = weight;
    if (bias) in[k++] = bias;
    Params p{};
    p.i[0] = normalized_ndim;
    p.i[1] = weight != nullptr;
    p.i[2] = bias != nullptr;
    p.f[0] = eps;
    return apply(&op_layer_norm, in, k, &p);
}
}

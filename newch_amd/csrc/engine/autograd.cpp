// Eager dispatch and tape-based reverse-mode autograd.  Reference: engine/src/autograd/autograd.c
// (nc__apply :12-82, nc_release_temp :95-105, nc_backward_ex :107-184) and gradcheck.c.
//
// Same contract as the reference: every op goes through apply(); a node is recorded when grad is
// enabled and an input requires grad; backward walks the tape newest to oldest, accumulates into
// grad buffers, and (unless RETAIN) frees each node's output grad and backward temporaries right
// after use, plus its forward activation with FREE_GRAPH.  Device memory is stream-ordered, so an
// arena block freed here may be handed to the next kernel at once.
#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include "engine.hpp"

namespace nce {

nc_tensor *apply(const OpDef *op, nc_tensor **in, int n_in, const Params *p) {
    for (int i = 0; i < n_in; i++)
        if (!in[i]) return nullptr;
    nc_ctx *ctx = in[0]->ctx;
    if (ctx->status != NC_OK) return nullptr;
    for (int i = 1; i < n_in; i++) {
        if (in[i]->ctx != ctx) {
            error(ctx, NC_ERR_ARG, "%s: inputs belong to different contexts", op->name);
            return nullptr;
        }
    }
    const bool persistent = persistent_mode(ctx);
    nc_node *n = (nc_node *)host_alloc(ctx, sizeof(nc_node), false);
    if (!n) return nullptr;
    n->op = op;
    n->n_in = n_in;
    for (int i = 0; i < n_in; i++) n->in[i] = in[i];
    if (p) n->p = *p;

    nc_dtype dt;
    int nd = 0;
    int64_t shape[NC_MAX_DIMS];
    if (op->infer(n, &dt, &nd, shape) != NC_OK) return nullptr;

    bool record = ctx->grad_enabled && !persistent && op->backward != nullptr;
    if (record) {
        record = false;
        for (int i = 0; i < n_in; i++)
            if (needs_grad(in[i])) record = true;
    }
    const bool can_view = op->view != nullptr && !persistent;
    if (!(can_view && op->view(n, nd, shape))) {
        n->out = tensor_new(ctx, dt, nd, shape, persistent);
        if (!n->out) return nullptr;
        // an unrecorded op never runs backward: whatever forward allocates besides the output is dead
        // once it returns (inference memory)
        const bool scratch = !record && !persistent && !ctx->bwd_logging;
        if (scratch) {
            ctx->bwd_logging = true;
            ctx->bwd_tmp.clear();
        }
        const nc_status st = op->forward(n);
        if (scratch) {
            ctx->bwd_logging = false;
            for (auto &b : ctx->bwd_tmp) arena_free(ctx, (char *)b.first, b.second);
            ctx->bwd_tmp.clear();
            n->saved = nullptr;
        }
        if (st != NC_OK) return nullptr;
        if (ctx->status != NC_OK) return nullptr;
    }
    if (!n->out) return nullptr;
    if (record) {
        for (int i = 0; i < n_in; i++) owner_of(in[i])->flags |= TF_ON_TAPE;
        owner_of(n->out)->flags |= TF_ON_TAPE;
        n->out->flags |= TF_REQUIRES_GRAD;
        n->out->node = n;
        n->prev = ctx->tape;
        ctx->tape = n;
    }
    return n->out;
}

}  // namespace nce

using namespace nce;

extern "C" {

nc_status nc_backward(nc_tensor *loss) { return nc_backward_ex(loss, 0, nullptr, 0); }

void nc_release_temp(nc_tensor *t) {
    if (!t || (t->flags & (TF_PERSISTENT | TF_ON_TAPE)) || !(t->flags & TF_OWNS_DATA) || !t->dev) return;
    nc_ctx *ctx = t->ctx;
    arena_free(ctx, t->dev, t->bytes);
    t->dev = nullptr;
    t->res = 0;
    if (t->grad && t->grad->dev && !(t->grad->flags & TF_PERSISTENT)) {
        arena_free(ctx, t->grad->dev, t->grad->bytes);
        t->grad->dev = nullptr;
        t->grad = nullptr;
    }
}

nc_status nc_backward_ex(nc_tensor *loss, int flags, nc_tensor *const *keep, int n_keep) {
    if (!loss) return NC_ERR_ARG;
    nc_ctx *ctx = loss->ctx;
    if (ctx->status != NC_OK) return ctx->status;
    if (nc_numel(loss) != 1 || loss->dtype != NC_F32) {
        error(ctx, NC_ERR_SHAPE, "backward: loss must be a single f32 element");
        return ctx->status;
    }
    if (!needs_grad(loss)) {
        error(ctx, NC_ERR_STATE,
              "backward: loss does not require grad (no parameter reached it, or grad was disabled)");
        return ctx->status;
    }
    // only nodes that lead to this loss take part
    const uint32_t ep = ++ctx->mark_epoch;
    if (loss->node) loss->node->mark = ep;
    for (nc_node *n = ctx->tape; n; n = n->prev) {
        if (n->mark != ep) continue;
        if (n->released) {
            error(ctx, NC_ERR_STATE,
                  "backward: part of this graph was released by an earlier backward "
                  "(use retain_graph=True on the first backward to run it twice)");
            return ctx->status;
        }
        for (int i = 0; i < n->n_in; i++)
            if (n->in[i]->node && needs_grad(n->in[i])) n->in[i]->node->mark = ep;
    }
    const bool retain = (flags & NC_BACKWARD_RETAIN) != 0;
    const bool free_graph = !retain && (flags & NC_BACKWARD_FREE_GRAPH);
    std::vector<const char *> kept;  // device storages that must survive (views share storage)
    if (free_graph)
        for (int i = 0; i < n_keep; i++)
            if (keep[i]) kept.push_back(owner_of(keep[i])->dev);
    std::sort(kept.begin(), kept.end());
    // intermediate grads start from zero (lazily: a fresh buffer is zero-filled if read before written)
    for (nc_node *n = ctx->tape; n; n = n->prev)
        if (n->mark == ep && n->out->grad) n->out->grad->flags |= TF_GRAD_FRESH;

    nc_tensor *g = grad_buf(loss);
    if (!g) return ctx->status;
    if (g->flags & TF_GRAD_FRESH) {
        if (!fill_zero(g)) return ctx->status;
    }
    if (!hip_layer_ok(ctx, nc_hip_add_scalar_at(fptr(g), 1.0f, ctx->stream), "backward seed")) return ctx->status;
    wrote_dev(g);

    for (nc_node *n = ctx->tape; n; n = n->prev) {
        if (n->mark != ep || !n->out->grad) continue;
        ctx->bwd_logging = !retain;
        ctx->bwd_tmp.clear();
        n->op->backward(n);
        ctx->bwd_logging = false;
        if (ctx->status != NC_OK) return ctx->status;
        if (retain) continue;
        for (auto &b : ctx->bwd_tmp) arena_free(ctx, (char *)b.first, b.second);
        ctx->bwd_tmp.clear();
        nc_tensor *o = n->out, *og = o->grad;
        if (og->dev && !(og->flags & TF_PERSISTENT)) arena_free(ctx, og->dev, og->bytes);
        og->dev = nullptr;
        o->grad = nullptr;
        if (free_graph && o != loss && (o->flags & TF_OWNS_DATA) && !(o->flags & TF_PERSISTENT) &&
            !std::binary_search(kept.begin(), kept.end(), (const char *)o->dev)) {
            arena_free(ctx, o->dev, o->bytes);
            o->dev = nullptr;
            o->res = 0;
            n->released = 1;
        }
    }
    return ctx->status;
}

void nc_zero_grad(nc_tensor *t) {
    if (t && t->grad && !(t->flags & TF_GRAD_CLEARED)) t->grad->flags |= TF_GRAD_FRESH;
}

void nc_clear_grad(nc_tensor *t) {
    if (t && t->grad) t->flags |= TF_GRAD_CLEARED;
}

float nc_gradcheck(nc_ctx *ctx, nc_scalar_fn fn, nc_tensor **inputs, int n_inputs, void *user, float eps) {
    for (int i = 0; i < n_inputs; i++) nc_zero_grad(inputs[i]);
    nc_tensor *y = fn(ctx, inputs, user);
    if (!y || nc_backward(y) != NC_OK) return INFINITY;
    float max_err = 0.0f;
    const int prev = nc_set_grad_enabled(ctx, 0);
    for (int i = 0; i < n_inputs && nc_ok(ctx); i++) {
        nc_tensor *x = inputs[i];
        if (!needs_grad(x)) continue;
        const int64_t n = nc_numel(x);
        if (!nc_data_f32(x)) {
            error(ctx, NC_ERR_ARG, "gradcheck: input %d must be contiguous f32", i);
            break;
        }
        std::vector<float> ana((size_t)n, 0.0f);
        if (x->grad && !nc_copy_to(x->grad, ana.data(), ana.size() * sizeof(float))) break;
        for (int64_t j = 0; j < n; j++) {
            float *d = nc_data_f32(x);  // re-taken: the host copy stays authoritative for the next op
            const float orig = d[j];
            d[j] = orig + eps;
            const float fp = nc_item(fn(ctx, inputs, user));
            d = nc_data_f32(x);
            d[j] = orig - eps;
            const float fm = nc_item(fn(ctx, inputs, user));
            d = nc_data_f32(x);
            d[j] = orig;
            const float num = (fp - fm) / (2.0f * eps);
            const float a = ana[(size_t)j];
            const float denom = fmaxf(1.0f, fmaxf(fabsf(num), fabsf(a)));
            const float err = fabsf(num - a) / denom;
            if (!(err <= max_err)) max_err = err;
        }
    }
    nc_set_grad_enabled(ctx, prev);
    return nc_ok(ctx) ? max_err : INFINITY;
}

}  // extern "C"

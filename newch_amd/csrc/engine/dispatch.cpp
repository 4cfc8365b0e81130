// Op dispatch, the tape and the backward pass.
//
// The contract is the reference's (engine/src/autograd/autograd.c, gradcheck.c): every op call goes
// through apply(); a call is recorded when grad is enabled, the op is differentiable and an input
// requires grad; nc_backward_ex walks the recorded calls that lead to the loss newest to oldest,
// accumulating into gradient buffers, and by default hands each node's output gradient back as soon
// as it has been passed on (FREE_GRAPH also its activation).  The machinery is this engine's own:
//   * an OpCall object runs one call: the shape rule, the output (a view when the op's alias rule
//     applies, else new storage), the forward inside a Scratch scope that returns the op's
//     temporaries when the forward ends, and the tape entry;
//   * the tape is a vector of nodes; a BackwardPass marks the nodes that reach the loss in one
//     reverse sweep over it, then runs their backward functions, each in a Scratch scope, and
//     applies its release policy (kept storages in a hash set);
//   * gradcheck perturbs one element at a time in device memory (a 4-byte write of the perturbed
//     value) instead of through a host mirror that the next op would re-upload whole.
// Device memory is stream-ordered, so any block handed back here may go to the next kernel at once.
#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <unordered_set>

#include "engine.hpp"

namespace nce {

// ---- scratch scopes --------------------------------------------------------------------------------
Scratch::Scratch(nc_ctx *ctx) : ctx_(ctx), outer_(ctx->scratch) { ctx->scratch = this; }

Scratch::~Scratch() {
    ctx_->scratch = outer_;
    for (auto &b : blocks_) arena_free(ctx_, b.first, b.second);
}

void Scratch::keep(const void *p) {
    for (auto &b : blocks_)
        if (b.first == p) {
            b = blocks_.back();
            blocks_.pop_back();
            return;
        }
}

void *save_state(nc_node *n, size_t bytes) {
    nc_ctx *ctx = n->in[0]->ctx;
    char *p = arena_alloc(ctx, bytes ? bytes : 1);
    if (!p) return nullptr;
    if (ctx->scratch) ctx->scratch->keep(p);
    n->saved = p;
    n->saved_bytes = bytes ? bytes : 1;
    return p;
}

static void drop_state(nc_node *n) {
    if (!n->saved) return;
    arena_free(n->in[0]->ctx, (char *)n->saved, n->saved_bytes);
    n->saved = nullptr;
}

// ---- one op call -----------------------------------------------------------------------------------
class OpCall {
  public:
    OpCall(const OpDef *op, nc_tensor **in, int n_in, const Params *p) : op_(op), in_(in), n_in_(n_in), p_(p) {}

    nc_tensor *run() {
        if (!inputs_usable()) return nullptr;
        nc_node *n = (nc_node *)host_alloc(ctx_, sizeof(nc_node), false);
        if (!n) return nullptr;
        n->op = op_;
        n->n_in = n_in_;
        std::copy(in_, in_ + n_in_, n->in);
        if (p_) n->p = *p_;
        OutSpec spec;
        if (op_->shape(n, spec) != NC_OK) return nullptr;
        const bool persistent = persistent_mode(ctx_);
        const bool record = recorded(persistent);
        // persistent results own their storage (each can be released alone): never views
        const bool viewed = !persistent && op_->alias && op_->alias(n, spec);
        if (!viewed && !materialize(n, spec, persistent, record)) return nullptr;
        if (!n->out) return nullptr;
        if (record) push(n);
        return n->out;
    }

  private:
    bool inputs_usable() {
        for (int i = 0; i < n_in_; i++)
            if (!in_[i]) return false;  // an earlier failure propagates as NULL
        ctx_ = in_[0]->ctx;
        if (ctx_->status != NC_OK) return false;
        for (int i = 1; i < n_in_; i++)
            if (in_[i]->ctx != ctx_) {
                error(ctx_, NC_ERR_ARG, "%s: inputs belong to different contexts", op_->name);
                return false;
            }
        return true;
    }

    bool recorded(bool persistent) const {
        if (!ctx_->grad_enabled || persistent || !op_->backward) return false;
        return std::any_of(in_, in_ + n_in_, [](const nc_tensor *t) { return needs_grad(t); });
    }

    // new storage for the output and the forward kernels; the call's temporaries go back when the
    // forward ends, and an unrecorded call's saved state with them (nothing will run its backward)
    bool materialize(nc_node *n, const OutSpec &spec, bool persistent, bool record) {
        n->out = tensor_new(ctx_, spec.dtype, spec.dims.rank, spec.dims.e, persistent);
        if (!n->out) return false;
        nc_status st;
        {
            Scratch scratch(ctx_);
            st = op_->forward(n);
        }
        if (!record) drop_state(n);
        return st == NC_OK && ctx_->status == NC_OK;
    }

    void push(nc_node *n) {
        // its backward reads these: their storage stays (owners, for views)
        for (int i = 0; i < n_in_; i++) owner_of(in_[i])->flags |= TF_ON_TAPE;
        owner_of(n->out)->flags |= TF_ON_TAPE;
        n->out->flags |= TF_REQUIRES_GRAD;
        n->out->node = n;
        n->seq = (uint32_t)ctx_->tape.size();
        ctx_->tape.push_back(n);
    }

    const OpDef *op_;
    nc_tensor **in_;
    int n_in_;
    const Params *p_;
    nc_ctx *ctx_ = nullptr;
};

nc_tensor *apply(const OpDef *op, nc_tensor **in, int n_in, const Params *p) {
    return OpCall(op, in, n_in, p).run();
}

// ---- the backward pass -----------------------------------------------------------------------------
class BackwardPass {
  public:
    BackwardPass(nc_tensor *loss, int flags) : loss_(loss), ctx_(loss->ctx) {
        retain_ = (flags & NC_BACKWARD_RETAIN) != 0;
        free_graph_ = !retain_ && (flags & NC_BACKWARD_FREE_GRAPH) != 0;
    }

    void keep(nc_tensor *const *keep, int n_keep) {
        if (!free_graph_) return;
        for (int i = 0; i < n_keep; i++)
            if (keep[i]) kept_.insert(owner_of(keep[i])->dev);
    }

    nc_status run() {
        if (!loss_ok() || !reach()) return ctx_->status;
        // intermediate gradients restart from zero (lazily); leaf gradients keep accumulating
        for (nc_node *n : live_)
            if (n->out->grad) n->out->grad->flags |= TF_GRAD_FRESH;
        if (!seed()) return ctx_->status;
        for (nc_node *n : live_) {
            if (!n->out->grad) continue;  // nothing reached this node's output
            {
                Scratch scratch(ctx_);
                n->op->backward(n);
            }
            if (ctx_->status != NC_OK) return ctx_->status;
            release(n);
        }
        return ctx_->status;
    }

  private:
    bool loss_ok() {
        if (nc_numel(loss_) != 1 || loss_->dtype != NC_F32) {
            error(ctx_, NC_ERR_SHAPE, "backward: loss must be a single f32 element");
            return false;
        }
        if (!needs_grad(loss_)) {
            error(ctx_, NC_ERR_STATE,
                  "backward: loss does not require grad (no parameter reached it, or grad was disabled)");
            return false;
        }
        return true;
    }

    // the nodes that lead to the loss, newest first: a node is on the path when its output is the
    // loss or feeds a node on the path through an input that requires grad
    bool reach() {
        const std::vector<nc_node *> &tape = ctx_->tape;
        std::vector<char> on(tape.size(), 0);
        // a node of this step's tape (a tensor kept past nc_step_end carries a stale one)
        auto taped = [&](const nc_node *n) { return n && n->seq < tape.size() && tape[n->seq] == n; };
        if (taped(loss_->node)) on[loss_->node->seq] = 1;
        for (size_t k = tape.size(); k-- > 0;) {
            if (!on[k]) continue;
            nc_node *n = tape[k];
            if (n->released) {
                error(ctx_, NC_ERR_STATE,
                      "backward: part of this graph was released by an earlier backward "
                      "(use retain_graph=True on the first backward to run it twice)");
                return false;
            }
            live_.push_back(n);
            for (int i = 0; i < n->n_in; i++) {
                const nc_tensor *x = n->in[i];
                if (taped(x->node) && needs_grad(x)) on[x->node->seq] = 1;
            }
        }
        return true;
    }

    // d loss / d loss = 1, added to the loss's gradient (a fresh buffer gets the 1 directly)
    bool seed() {
        nc_tensor *g = grad_buf(loss_);
        if (!g) return false;
        if (g->flags & TF_GRAD_FRESH) {
            g->flags &= ~TF_GRAD_FRESH;
            char *p = dptr(g);
            if (!p || !hip_layer_ok(ctx_, nc_hip_fill(p, 4, 0x3f800000u, 1, ctx_->stream), "backward seed"))
                return false;
        } else if (!hip_layer_ok(ctx_, nc_hip_add_scalar_at(fptr(g), 1.0f, ctx_->stream), "backward seed")) {
            return false;
        }
        wrote_dev(g);
        return true;
    }

    // after a node's backward: its output gradient has been passed on; with FREE_GRAPH its
    // activation is dead too (every consumer's backward ran before it), unless the caller keeps it
    void release(nc_node *n) {
        if (retain_) return;
        nc_tensor *o = n->out, *og = o->grad;
        if (og->dev && !(og->flags & TF_PERSISTENT)) arena_free(ctx_, og->dev, og->bytes);
        og->dev = nullptr;
        o->grad = nullptr;
        if (!free_graph_ || o == loss_ || !(o->flags & TF_OWNS_DATA) || (o->flags & TF_PERSISTENT) ||
            kept_.count(o->dev))
            return;
        arena_free(ctx_, o->dev, o->bytes);
        o->dev = nullptr;
        o->res = 0;
        n->released = true;
        drop_state(n);
    }

    nc_tensor *loss_;
    nc_ctx *ctx_;
    bool retain_ = false, free_graph_ = false;
    std::unordered_set<const char *> kept_;
    std::vector<nc_node *> live_;  // newest first
};

// ---- numerical gradient check ----------------------------------------------------------------------
// x[j] = v in device memory (x contiguous); the device copy becomes the authoritative one
static bool poke(nc_tensor *x, int64_t j, float v) {
    nc_ctx *ctx = x->ctx;
    char *d = dptr(x);
    if (!d) return false;
    if (!hip_ok(ctx, hipMemcpyAsync(d + 4 * j, &v, 4, hipMemcpyHostToDevice, ctx->stream), "gradcheck") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "gradcheck"))
        return false;
    wrote_dev(x);
    return true;
}

static float relative_gap(float num, float ana) {
    return fabsf(num - ana) / fmaxf(1.0f, fmaxf(fabsf(num), fabsf(ana)));
}

}  // namespace nce

using namespace nce;

extern "C" {

nc_status nc_backward(nc_tensor *loss) { return nc_backward_ex(loss, 0, nullptr, 0); }

nc_status nc_backward_ex(nc_tensor *loss, int flags, nc_tensor *const *keep, int n_keep) {
    if (!loss) return NC_ERR_ARG;
    if (loss->ctx->status != NC_OK) return loss->ctx->status;
    BackwardPass pass(loss, flags);
    pass.keep(keep, n_keep);
    return pass.run();
}

void nc_release_temp(nc_tensor *t) {
    if (!t || (t->flags & (TF_PERSISTENT | TF_ON_TAPE)) || !(t->flags & TF_OWNS_DATA) || !t->dev) return;
    nc_ctx *ctx = t->ctx;
    arena_free(ctx, t->dev, t->bytes);
    t->dev = nullptr;
    t->res = 0;
    nc_tensor *g = t->grad;
    if (g && g->dev && !(g->flags & TF_PERSISTENT)) {
        arena_free(ctx, g->dev, g->bytes);
        g->dev = nullptr;
        t->grad = nullptr;
    }
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
    float worst = 0.0f;
    const int was = nc_set_grad_enabled(ctx, 0);
    for (int i = 0; i < n_inputs && nc_ok(ctx); i++) {
        nc_tensor *x = inputs[i];
        if (!needs_grad(x)) continue;
        if (x->dtype != NC_F32 || !nc_is_contiguous(x)) {
            error(ctx, NC_ERR_ARG, "gradcheck: input %d must be contiguous f32", i);
            break;
        }
        const size_t n = (size_t)nc_numel(x);
        std::vector<float> at(n), ana(n, 0.0f);  // the point, and the analytic gradient there
        if (!nc_copy_to(x, at.data(), n * sizeof(float))) break;
        if (x->grad && !nc_copy_to(x->grad, ana.data(), n * sizeof(float))) break;
        for (size_t j = 0; j < n && nc_ok(ctx); j++) {
            const float v = at[j];
            if (!poke(x, (int64_t)j, v + eps)) break;
            const float up = nc_item(fn(ctx, inputs, user));
            if (!poke(x, (int64_t)j, v - eps)) break;
            const float down = nc_item(fn(ctx, inputs, user));
            if (!poke(x, (int64_t)j, v)) break;
            const float gap = relative_gap((up - down) / (2.0f * eps), ana[j]);
            if (!(gap <= worst)) worst = gap;  // a NaN gap wins
        }
    }
    nc_set_grad_enabled(ctx, was);
    return nc_ok(ctx) ? worst : INFINITY;
}

}  // extern "C"

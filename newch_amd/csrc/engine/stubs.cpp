// The rest of the reference ABI (engine/include/nc.h) outside this engine's hot path: convolution,
// pooling, masking and modules.  Every symbol exists, so the
// reference's ctypes bindings resolve all their names at import (newch/_lib.py:174-177), and every
// call fails cleanly the reference way -- a sticky NC_ERR_STATE in the context and a NULL / error
// result -- instead of computing anything on the host.
#include "engine.hpp"

using namespace nce;

static nc_tensor *absent(nc_tensor *any, const char *name) {
    if (any) error(any->ctx, NC_ERR_STATE, "%s: not in this engine (the MI355X engine runs the elementwise, "
                                          "reduction, normalization, loss, optimizer, linear-algebra and int8 ops)", name);
    return nullptr;
}

static void absent_ctx(nc_ctx *ctx, const char *name) {
    if (ctx) error(ctx, NC_ERR_STATE, "%s: not in this engine", name);
}

extern "C" {

nc_tensor *nc_index_select(nc_tensor *x, nc_tensor *) { return absent(x, "index_select"); }
nc_tensor *nc_conv2d(nc_tensor *x, nc_tensor *, nc_tensor *, int, int, int, int) { return absent(x, "conv2d"); }
nc_tensor *nc_conv2d_ex(nc_tensor *x, nc_tensor *, nc_tensor *, int, int, int, int, int, int, int) {
    return absent(x, "conv2d");
}
nc_tensor *nc_max_pool2d(nc_tensor *x, int, int, int, int, int, int) { return absent(x, "max_pool2d"); }
nc_tensor *nc_avg_pool2d(nc_tensor *x, int, int, int, int, int, int) { return absent(x, "avg_pool2d"); }
nc_tensor *nc_dropout(nc_tensor *x, float) { return absent(x, "dropout"); }
nc_tensor *nc_batch_norm(nc_tensor *x, nc_tensor *, nc_tensor *, nc_tensor *, nc_tensor *, int, float, float) {
    return absent(x, "batch_norm");
}
nc_tensor *nc_masked_fill(nc_tensor *x, nc_tensor *, float) { return absent(x, "masked_fill"); }
nc_tensor *nc_compare(nc_tensor *a, nc_tensor *b, nc_cmp) { return absent(a ? a : b, "compare"); }
nc_tensor *nc_cat(int n, nc_tensor *const *xs, int) { return absent(n > 0 && xs ? xs[0] : nullptr, "cat"); }


nc_module *nc_linear(nc_ctx *ctx, int64_t, int64_t, int) {
    absent_ctx(ctx, "nc_linear");
    return nullptr;
}
nc_module *nc_act(nc_ctx *ctx, nc_activation) {
    absent_ctx(ctx, "nc_act");
    return nullptr;
}
nc_module *nc_sequential(nc_ctx *ctx, int, nc_module **) {
    absent_ctx(ctx, "nc_sequential");
    return nullptr;
}
nc_tensor *nc_forward(nc_module *, nc_tensor *x) { return absent(x, "nc_forward"); }
int nc_parameters(nc_module *, nc_tensor **, int) { return 0; }
const char *nc_module_name(const nc_module *) { return ""; }
void nc_set_training(nc_module *, int) {}

}  // extern "C"

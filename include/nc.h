/*
 * nc.h -- public C API of the newch engine, MI355X build (newch_amd/libnc.so).
 *
 * Drop-in ABI: every function, enum value and struct layout below matches the reference engine's
 * public header (engine/include/nc.h, version 0.4.0), which its ctypes bindings bind by name
 * (newch/_lib.py:78-177) and which C programs link against.  Tensors live in HBM on one HIP device;
 * host-visible accessors (nc_data_f32, nc_item, nc_get, nc_copy_to, nc_print) synchronise and copy
 * back, host writes (nc_copy_from, writes through nc_data_f32) are uploaded before the next op.
 * Ops on the hot path run hand-written gfx950 kernels (include/nc_hip.h); the other ops of the
 * reference API exist as symbols and fail cleanly with NC_ERR_STATE ("not in this engine").
 *
 * Memory and error model as the reference: persistent tensors live until nc_free_ctx / nc_release;
 * temporaries live in the step arena (here a device bump arena) until nc_step_end; ops never abort,
 * the first error sticks in the context and every op propagates NULL.
 */
#ifndef NC_H
#define NC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NC_API __attribute__((visibility("default")))

#define NC_VERSION_MAJOR 0
#define NC_VERSION_MINOR 4
#define NC_VERSION_PATCH 0

#define NC_MAX_DIMS 6
#define NC_ALL_AXES (-128) /* reduce over every axis */

typedef enum { NC_F32 = 0, NC_I32 = 1, NC_F16 = 2, NC_I8 = 3, NC_U8 = 4, NC_DTYPE_COUNT } nc_dtype;
typedef enum { NC_DEVICE_CPU = 0 } nc_device;
typedef enum { NC_OK = 0, NC_ERR_SHAPE = 1, NC_ERR_DTYPE = 2, NC_ERR_OOM = 3, NC_ERR_ARG = 4, NC_ERR_STATE = 5 } nc_status;

typedef struct nc_ctx nc_ctx;
typedef struct nc_tensor nc_tensor;
typedef struct nc_module nc_module;
typedef struct nc_optim nc_optim;

/* ---- context (reference nc.h:78-117) --------------------------------------------------------- */
typedef struct {
    size_t arena_chunk_bytes; /* device step-arena growth unit; 0 = 64 MiB here */
    uint64_t seed;            /* RNG seed; 0 = fixed default */
    int force_reference;      /* accepted for compatibility; the device kernels have one tier */
    int threads;              /* host threads for host-side work (0 = all cores, capped at 64) */
} nc_config;

NC_API nc_ctx *nc_init(const nc_config *cfg);
NC_API void nc_free_ctx(nc_ctx *ctx);
NC_API void nc_manual_seed(nc_ctx *ctx, uint64_t seed);
NC_API void nc_step_end(nc_ctx *ctx);
NC_API void nc_arena_trim(nc_ctx *ctx);
NC_API int nc_num_threads(const nc_ctx *ctx);
NC_API void nc_persistent_begin(nc_ctx *ctx);
NC_API void nc_persistent_end(nc_ctx *ctx);
NC_API int nc_set_grad_enabled(nc_ctx *ctx, int enabled);
NC_API int nc_ok(const nc_ctx *ctx);
NC_API nc_status nc_status_code(const nc_ctx *ctx);
NC_API const char *nc_error(const nc_ctx *ctx);
NC_API void nc_clear_error(nc_ctx *ctx);

typedef struct {
    size_t persistent_bytes;     /* device bytes of persistent tensors */
    size_t arena_bytes_in_use;   /* device step-arena bytes handed out */
    size_t arena_bytes_reserved; /* device step-arena bytes held */
    size_t arena_peak_bytes;
} nc_mem_stats;

NC_API nc_mem_stats nc_get_mem_stats(const nc_ctx *ctx);
NC_API void nc_reset_peak(nc_ctx *ctx);

/* ---- platform (reference nc.h:123-136) --------------------------------------------------------- */
typedef struct {
    const char *arch;
    int has_neon;
    int has_dotprod;
    int has_fp16;
    int has_avx2;
    int has_fma;
    int has_rvv;
    int n_cores;
    int n_big_cores;
} nc_cpu_info;

NC_API const nc_cpu_info *nc_cpu(const nc_ctx *ctx);
NC_API const char *nc_kernel_backend(const nc_ctx *ctx); /* "hip:gfx950" */

/* ---- tensors (reference nc.h:142-186) ------------------------------------------------------------ */
NC_API nc_tensor *nc_empty(nc_ctx *ctx, nc_dtype dt, int ndim, const int64_t *shape);
NC_API nc_tensor *nc_zeros(nc_ctx *ctx, nc_dtype dt, int ndim, const int64_t *shape);
NC_API nc_tensor *nc_full(nc_ctx *ctx, float value, int ndim, const int64_t *shape);
NC_API nc_tensor *nc_randn(nc_ctx *ctx, float stddev, int ndim, const int64_t *shape);
NC_API nc_tensor *nc_rand_uniform(nc_ctx *ctx, float lo, float hi, int ndim, const int64_t *shape);
NC_API nc_tensor *nc_from_data(nc_ctx *ctx, nc_dtype dt, const void *data, int ndim, const int64_t *shape);
NC_API nc_tensor *nc_scalar(nc_ctx *ctx, float value);
NC_API nc_tensor *nc_parameter(nc_ctx *ctx, const nc_tensor *init, int ndim, const int64_t *shape);

NC_API int nc_ndim(const nc_tensor *t);
NC_API int64_t nc_dim(const nc_tensor *t, int axis);
NC_API const int64_t *nc_shape(const nc_tensor *t);
NC_API int64_t nc_numel(const nc_tensor *t);
NC_API nc_dtype nc_get_dtype(const nc_tensor *t);
NC_API int nc_is_contiguous(const nc_tensor *t);
NC_API int nc_requires_grad(const nc_tensor *t);
NC_API int nc_is_persistent(const nc_tensor *t);
NC_API void nc_release(nc_tensor *t);
NC_API void nc_set_requires_grad(nc_tensor *t, int on);
NC_API nc_tensor *nc_grad(const nc_tensor *t);
NC_API void nc_set_name(nc_tensor *t, const char *name);
NC_API const char *nc_name(const nc_tensor *t);

/* Host views of device data: the pointer stays valid until the tensor is released; taking it makes
 * the host copy authoritative (the device copy is refreshed from it before the next device use). */
NC_API float *nc_data_f32(nc_tensor *t);
NC_API int32_t *nc_data_i32(nc_tensor *t);
NC_API float nc_item(const nc_tensor *t);
NC_API float nc_get(const nc_tensor *t, const int64_t *index);
NC_API int nc_copy_to(const nc_tensor *t, void *dst, size_t dst_bytes);
NC_API int nc_copy_from(nc_tensor *t, const void *src, size_t src_bytes);
NC_API void nc_print(const nc_tensor *t);

/* ---- ops (reference nc.h:192-287) ------------------------------------------------------------------ */
NC_API nc_tensor *nc_add(nc_tensor *a, nc_tensor *b);
NC_API nc_tensor *nc_sub(nc_tensor *a, nc_tensor *b);
NC_API nc_tensor *nc_mul(nc_tensor *a, nc_tensor *b);
NC_API nc_tensor *nc_div(nc_tensor *a, nc_tensor *b);

NC_API nc_tensor *nc_neg(nc_tensor *x);
NC_API nc_tensor *nc_exp(nc_tensor *x);
NC_API nc_tensor *nc_log(nc_tensor *x);
NC_API nc_tensor *nc_sqrt(nc_tensor *x);
NC_API nc_tensor *nc_relu(nc_tensor *x);
NC_API nc_tensor *nc_sigmoid(nc_tensor *x);
NC_API nc_tensor *nc_tanh(nc_tensor *x);
NC_API nc_tensor *nc_scale(nc_tensor *x, float s);
NC_API nc_tensor *nc_add_scalar(nc_tensor *x, float s);
NC_API nc_tensor *nc_pow_scalar(nc_tensor *x, float p);

NC_API nc_tensor *nc_leaky_relu(nc_tensor *x, float negative_slope);
NC_API nc_tensor *nc_relu6(nc_tensor *x);
NC_API nc_tensor *nc_hardsigmoid(nc_tensor *x);
NC_API nc_tensor *nc_hardswish(nc_tensor *x);
NC_API nc_tensor *nc_silu(nc_tensor *x);
NC_API nc_tensor *nc_gelu(nc_tensor *x, int approximate_tanh);

NC_API nc_tensor *nc_matmul(nc_tensor *a, nc_tensor *b);
NC_API nc_tensor *nc_linear_fn(nc_tensor *x, nc_tensor *weight, nc_tensor *bias);

NC_API nc_tensor *nc_sum(nc_tensor *x, int axis, int keepdim);
NC_API nc_tensor *nc_mean(nc_tensor *x, int axis, int keepdim);
NC_API nc_tensor *nc_max(nc_tensor *x, int axis, int keepdim);

NC_API nc_tensor *nc_reshape(nc_tensor *x, int ndim, const int64_t *shape);
NC_API nc_tensor *nc_transpose(nc_tensor *x, int axis0, int axis1);
NC_API nc_tensor *nc_slice(nc_tensor *x, int axis, int64_t start, int64_t length, int64_t step);
NC_API nc_tensor *nc_contiguous(nc_tensor *x);
NC_API nc_tensor *nc_index_select(nc_tensor *x, nc_tensor *idx);

NC_API nc_tensor *nc_conv2d(nc_tensor *x, nc_tensor *weight, nc_tensor *bias, int stride_h, int stride_w, int pad_h,
                            int pad_w);
NC_API nc_tensor *nc_conv2d_ex(nc_tensor *x, nc_tensor *weight, nc_tensor *bias, int stride_h, int stride_w,
                               int pad_h, int pad_w, int dilation_h, int dilation_w, int groups);
NC_API nc_tensor *nc_max_pool2d(nc_tensor *x, int k_h, int k_w, int stride_h, int stride_w, int pad_h, int pad_w);
NC_API nc_tensor *nc_avg_pool2d(nc_tensor *x, int k_h, int k_w, int stride_h, int stride_w, int pad_h, int pad_w);
NC_API nc_tensor *nc_dropout(nc_tensor *x, float p);
NC_API nc_tensor *nc_batch_norm(nc_tensor *x, nc_tensor *weight, nc_tensor *bias, nc_tensor *running_mean,
                                nc_tensor *running_var, int training, float momentum, float eps);

NC_API nc_tensor *nc_log_softmax(nc_tensor *x);
NC_API nc_tensor *nc_softmax(nc_tensor *x);
NC_API nc_tensor *nc_layer_norm(nc_tensor *x, int normalized_ndim, nc_tensor *weight, nc_tensor *bias, float eps);
NC_API nc_tensor *nc_masked_fill(nc_tensor *x, nc_tensor *mask, float value);
NC_API nc_tensor *nc_cross_entropy(nc_tensor *logits, nc_tensor *labels);
NC_API nc_tensor *nc_mse_loss(nc_tensor *pred, nc_tensor *target);
NC_API nc_tensor *nc_nll_loss(nc_tensor *logp, nc_tensor *labels, int sum);

NC_API nc_tensor *nc_argmax(nc_tensor *x, int axis);
NC_API nc_tensor *nc_detach(nc_tensor *x);

typedef enum { NC_CMP_EQ, NC_CMP_NE, NC_CMP_LT, NC_CMP_LE, NC_CMP_GT, NC_CMP_GE } nc_cmp;
NC_API nc_tensor *nc_compare(nc_tensor *a, nc_tensor *b, nc_cmp op);
NC_API nc_tensor *nc_cat(int n, nc_tensor *const *xs, int axis);
NC_API nc_tensor *nc_to_dtype(nc_tensor *x, nc_dtype dt);

/* ---- quantization (reference nc.h:295-298) ----------------------------------------------------- */
NC_API nc_tensor *nc_quantize_rows(nc_tensor *w, nc_tensor **scale);
NC_API nc_tensor *nc_linear_int8(nc_tensor *x, nc_tensor *wq, nc_tensor *w_scale, nc_tensor *bias);

/* ---- serialization (reference nc.h:305-307) ---------------------------------------------------- */
NC_API nc_status nc_save(nc_ctx *ctx, const char *path, int n, const char *const *names, nc_tensor *const *tensors);
NC_API nc_status nc_load(nc_ctx *ctx, const char *path, int n, const char *const *names, nc_tensor *const *tensors);

/* ---- autograd (reference nc.h:315-346) --------------------------------------------------------- */
NC_API nc_status nc_backward(nc_tensor *loss);
enum { NC_BACKWARD_FREE_GRAPH = 1, NC_BACKWARD_RETAIN = 2 };
NC_API void nc_release_temp(nc_tensor *t);
NC_API nc_status nc_backward_ex(nc_tensor *loss, int flags, nc_tensor *const *keep, int n_keep);
NC_API void nc_zero_grad(nc_tensor *t);
NC_API void nc_clear_grad(nc_tensor *t);
typedef nc_tensor *(*nc_scalar_fn)(nc_ctx *ctx, nc_tensor **inputs, void *user);
NC_API float nc_gradcheck(nc_ctx *ctx, nc_scalar_fn fn, nc_tensor **inputs, int n_inputs, void *user, float eps);

/* ---- modules and optimizers (reference nc.h:352-416; not in this engine) ------------------------ */
typedef enum { NC_ACT_RELU, NC_ACT_SIGMOID, NC_ACT_TANH } nc_activation;
NC_API nc_module *nc_linear(nc_ctx *ctx, int64_t in_features, int64_t out_features, int bias);
NC_API nc_module *nc_act(nc_ctx *ctx, nc_activation kind);
NC_API nc_module *nc_sequential(nc_ctx *ctx, int n, nc_module **mods);
NC_API nc_tensor *nc_forward(nc_module *m, nc_tensor *x);
NC_API int nc_parameters(nc_module *m, nc_tensor **out, int max);
NC_API const char *nc_module_name(const nc_module *m);
NC_API void nc_set_training(nc_module *m, int training);

typedef struct {
    float lr;
    float momentum;
    float weight_decay;
    float beta1, beta2, eps;
} nc_optim_opts;

NC_API nc_optim *nc_sgd(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts);
NC_API nc_optim *nc_adam(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts);
NC_API nc_optim *nc_adamw(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts);
NC_API nc_optim *nc_rmsprop(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts, int eps_inside_sqrt);
NC_API void nc_optim_zero_grad(nc_optim *o);
NC_API void nc_optim_clear_grad(nc_optim *o);
NC_API void nc_optim_step(nc_optim *o);
NC_API void nc_optim_free(nc_optim *o);
NC_API void nc_optim_set_lr(nc_optim *o, float lr);
NC_API float *nc_optim_state(nc_optim *o, int param, int slot);
NC_API int64_t nc_optim_get_step(const nc_optim *o);
NC_API void nc_optim_set_step(nc_optim *o, int64_t t);
NC_API void nc_optim_set_opts(nc_optim *o, nc_optim_opts opts);
NC_API void nc_optim_set_accumulation(nc_optim *o, int steps);
NC_API float nc_clip_grad_norm(nc_tensor **params, int n, float max_norm);

/* ---- device extensions of this engine (additive; the reference bindings never call them) -------- */
/* Number of visible HIP devices.  The device of a context is chosen at nc_init from the environment
 * variable NC_DEVICE ("hip:N" or "N", default 0) or later with nc_set_device (before any tensor). */
NC_API int nc_device_count(void);
NC_API int nc_set_device(nc_ctx *ctx, int device);
NC_API int nc_get_device(const nc_ctx *ctx);
/* Stream the context enqueues on (a hipStream_t; NULL = the context's own stream). */
NC_API void nc_set_stream(nc_ctx *ctx, void *stream);
NC_API void *nc_get_stream(const nc_ctx *ctx);
/* Waits for the context's queued device work; returns NC_OK or the first device error. */
NC_API nc_status nc_synchronize(nc_ctx *ctx);
/* Device address of a tensor's element 0 (NULL if it has no device storage). */
NC_API void *nc_device_ptr(nc_tensor *t);
/* A new tensor copied from device memory (device-to-device). */
NC_API nc_tensor *nc_from_device(nc_ctx *ctx, nc_dtype dt, const void *device_data, int ndim, const int64_t *shape);
/* Device allocations (hipMalloc calls) the context has made so far: arena chunks, large arena blocks
 * and persistent tensors.  Constant across steady-state steps, whose temporaries come from the arena. */
NC_API uint64_t nc_device_alloc_count(const nc_ctx *ctx);

#ifdef __cplusplus
}
#endif
#endif /* NC_H */

// Broadcast binary ops and their sum-to-shape gradients, strided copies, fills, conversions.
//
// Reference: ops_elementwise.c:19-54 (row functions), :108-186 (binary_fwd / binary_bwd),
// tensor.c:313-373 (nc__iterate, nc__copy_strided), ops_shape.c:474-504 (to_dtype).
//
// The reference walks every broadcast with a serial odometer, one indirect call per innermost row.
// Here the host coalesces dims (adjacent dims that are contiguous for every operand merge, size-1
// dims vanish) and each lane computes its operand offsets with multiply-high divisions; when the
// innermost output dim is unit-stride and a multiple of 4 long, a lane produces 4 outputs with one
// 128-bit store and loads every operand as a 128-bit vector (unit stride), a splat (stride 0) or a
// 4-element gather (any other stride).
//
// Gradients that are not reduced (an operand with the output's shape) are computed with the
// reference's fp32 expressions and are bit-identical to it.  Reduced gradients (sum-to-shape) are
// accumulated in fp64 over a fixed partition: partial sums per (kept index, chunk) then a fixed-order
// combine, so the result does not depend on scheduling.
#include "common.hpp"
#include "intdiv.hpp"

#include <stdlib.h>
#include <string.h>

#include <algorithm>

namespace nchip {

constexpr int kB = 256;

// ------------------------------------------------------------------------------------------------
// index maps
// ------------------------------------------------------------------------------------------------
template <int NOPS>
struct IdxMap {
    int nd;
    uint32_t size[NC_HIP_MAX_DIMS];  // innermost dim counted in work units (elements or vectors)
    IntDiv div[NC_HIP_MAX_DIMS];
    int64_t st[NOPS][NC_HIP_MAX_DIMS];  // element strides; innermost already multiplied by the unit
};

// offsets of every operand for work item w (row-major, last dim fastest)
template <int NOPS>
__device__ __forceinline__ void offsets(const IdxMap<NOPS> &m, uint32_t w, int64_t *off) {
#pragma unroll
    for (int o = 0; o < NOPS; o++) off[o] = 0;
#pragma unroll
    for (int d = NC_HIP_MAX_DIMS - 1; d >= 0; d--) {
        if (d < m.nd) {
            const uint32_t q = m.div[d].div(w);
            const uint32_t i = w - q * m.size[d];
            w = q;
#pragma unroll
            for (int o = 0; o < NOPS; o++) off[o] += (int64_t)i * m.st[o][d];
        }
    }
}

// loads 4 consecutive (along the innermost dim) elements of an operand with inner stride `is`
__device__ __forceinline__ f4 load4(const float *p, int64_t is, int mode) {
    if (mode == 1) return *(const f4 *)p;
    if (mode == 0) {
        const float v = *p;
        return f4{v, v, v, v};
    }
    return f4{p[0], p[is], p[2 * is], p[3 * is]};
}

template <int OP>
__device__ __forceinline__ float bin(float x, float y) {
    if constexpr (OP == NC_HIP_BIN_ADD) return x + y;
    else if constexpr (OP == NC_HIP_BIN_SUB) return x - y;
    else if constexpr (OP == NC_HIP_BIN_MUL) return x * y;
    else return x / y;
}

struct VecModes {
    int a, b;          // 0 splat, 1 vector, 2 gather
    int64_t ia, ib;    // inner element strides (for gathers)
};

// NC_BIN_UNROLL work items per lane are decoded and loaded before any is computed and stored, so
// several operand loads (mostly L2 hits on the broadcast operands) are in flight per lane; one wave
// per workgroup and a grid over the whole output (measured on MI355X, with the broadcast operand
// warmed first: 717-745 us for 2^30 outputs against 791 us for a CU-sized grid-stride grid).
#ifndef NC_BIN_UNROLL
#define NC_BIN_UNROLL 4
#endif
#ifndef NC_BIN_GRID_PER_CU
#define NC_BIN_GRID_PER_CU 65536
#endif
#ifndef NC_BIN_NT_STORE
#define NC_BIN_NT_STORE 1
#endif
#ifndef NC_BIN_WARM
#define NC_BIN_WARM 1  // warm dense broadcast operands before the kernels that re-read them
#endif
#ifndef NC_BIN_BLOCK
#define NC_BIN_BLOCK 64
#endif
#ifndef NC_BIN_SMALL_INDEX
#define NC_BIN_SMALL_INDEX 1  // 32-bit index kernel where offsets allow it
#endif
constexpr int kBU = NC_BIN_UNROLL;
constexpr int kBF = NC_BIN_BLOCK;  // forward workgroup size

template <int OP, bool VEC>
__global__ __launch_bounds__(kBF) void k_binary_fwd(const float *__restrict__ a, const float *__restrict__ b,
                                                    float *__restrict__ o, IdxMap<3> m, VecModes vm, uint32_t nwork) {
    const uint64_t step = (uint64_t)gridDim.x * kBF * kBU;
    for (uint64_t base = (uint64_t)blockIdx.x * kBF * kBU + threadIdx.x; base < nwork; base += step) {
        if constexpr (VEC) {
            f4 x[kBU], y[kBU];
            int64_t oo[kBU];
#pragma unroll
            for (int u = 0; u < kBU; u++) {
                const uint64_t w = base + (uint64_t)u * kBF;
                if (w < nwork) {
                    int64_t off[3];
                    offsets<3>(m, (uint32_t)w, off);
                    x[u] = load4(a + off[0], vm.ia, vm.a);
                    y[u] = load4(b + off[1], vm.ib, vm.b);
                    oo[u] = off[2];
                }
            }
#pragma unroll
            for (int u = 0; u < kBU; u++) {
                const uint64_t w = base + (uint64_t)u * kBF;
                if (w < nwork) {
                    f4 r;
                    r.x = bin<OP>(x[u].x, y[u].x);
                    r.y = bin<OP>(x[u].y, y[u].y);
                    r.z = bin<OP>(x[u].z, y[u].z);
                    r.w = bin<OP>(x[u].w, y[u].w);
                    if constexpr (NC_BIN_NT_STORE) __builtin_nontemporal_store(r, (f4 *)(o + oo[u]));
                    else *(f4 *)(o + oo[u]) = r;
                }
            }
        } else {
            float x[kBU], y[kBU];
            int64_t oo[kBU];
#pragma unroll
            for (int u = 0; u < kBU; u++) {
                const uint64_t w = base + (uint64_t)u * kBF;
                if (w < nwork) {
                    int64_t off[3];
                    offsets<3>(m, (uint32_t)w, off);
                    x[u] = a[off[0]];
                    y[u] = b[off[1]];
                    oo[u] = off[2];
                }
            }
#pragma unroll
            for (int u = 0; u < kBU; u++) {
                const uint64_t w = base + (uint64_t)u * kBF;
                if (w < nwork) o[oo[u]] = bin<OP>(x[u], y[u]);
            }
        }
    }
}

// 32-bit index path: fewer than 2^31 work items, at most 4 dims after coalescing, non-negative
// strides and every operand's largest element offset below 2^31.  The multiply-high division then
// needs no 64-bit add (quotient estimate + dividend < 2^32), the outermost index needs no division,
// offsets are 32-bit sums, and when every size, stride and quotient fits in 24 bits the products are
// full-rate 24-bit multiplies.  Only the uniform kernel arguments that ND dims use are passed, so the
// decode stays in scalar registers instead of spilling them.
template <int ND>
struct SmallMap {
    uint32_t size[ND];
    uint32_t mul[ND];
    uint32_t shift[ND];
    uint32_t st[3][ND];  // element strides; innermost already multiplied by the unit
};

struct SmallModes {
    int a, b;        // 0 splat, 1 vector, 2 gather, 3 vector read once (no broadcast dim)
    uint32_t ia, ib; // inner element strides (for gathers)
};

template <bool U24>
__device__ __forceinline__ uint32_t umul(uint32_t x, uint32_t y) {
    if constexpr (U24) return __umul24(x, y);
    else return x * y;
}

template <int ND, bool U24>
__device__ __forceinline__ void offsets_small(const SmallMap<ND> &m, uint32_t w, uint32_t *off) {
    off[0] = off[1] = off[2] = 0;
#pragma unroll
    for (int d = ND - 1; d >= 1; d--) {
        const uint32_t q = IntDiv::div31(w, m.mul[d], m.shift[d]);
        const uint32_t i = w - umul<U24>(q, m.size[d]);
        w = q;
#pragma unroll
        for (int o = 0; o < 3; o++) off[o] += umul<U24>(i, m.st[o][d]);
    }
#pragma unroll
    for (int o = 0; o < 3; o++) off[o] += umul<U24>(w, m.st[o][0]);
}

__device__ __forceinline__ f4 load4s(const float *p, uint32_t is, int mode) {
    if (mode == 3) return __builtin_nontemporal_load((const f4 *)p);  // read once: streamed past the caches
    if (mode == 1) return *(const f4 *)p;
    if (mode == 0) {
        const float v = *p;
        return f4{v, v, v, v};
    }
    return f4{p[0], p[is], p[2 * is], p[3 * is]};
}

// Launch shape of the 32-bit index kernel per op (a[64,512,1,64] op b[512,64] into 2^30 outputs):
// add, sub and mul run two work items per lane in 128-lane workgroups (685 -> 640 us against four
// in 64-lane ones); divide, with ten times the arithmetic per element, keeps four in 64-lane ones
// (660 us; 740 us with two in 128).
#ifndef NC_BIN_S_UNROLL
#define NC_BIN_S_UNROLL 2
#endif
#ifndef NC_BIN_S_BLOCK
#define NC_BIN_S_BLOCK 128
#endif
#ifndef NC_BIN_S_DIV_UNROLL
#define NC_BIN_S_DIV_UNROLL 4
#endif
#ifndef NC_BIN_S_DIV_BLOCK
#define NC_BIN_S_DIV_BLOCK 64
#endif
template <int OP>
constexpr int small_unroll() { return OP == NC_HIP_BIN_DIV ? NC_BIN_S_DIV_UNROLL : NC_BIN_S_UNROLL; }
template <int OP>
constexpr int small_block() { return OP == NC_HIP_BIN_DIV ? NC_BIN_S_DIV_BLOCK : NC_BIN_S_BLOCK; }

template <int OP, int ND, bool U24>
__global__ __launch_bounds__(small_block<OP>()) void k_binary_fwd_s(const float *__restrict__ a,
                                                                    const float *__restrict__ b,
                                                                    float *__restrict__ o, SmallMap<ND> m,
                                                                    SmallModes vm, uint32_t nwork) {
    constexpr int kU = small_unroll<OP>(), kBk = small_block<OP>();
    const uint32_t step = gridDim.x * kBk * kU;
    for (uint32_t base = blockIdx.x * kBk * kU + threadIdx.x; base < nwork; base += step) {
        f4 x[kU], y[kU];
        uint32_t oo[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const uint32_t w = base + u * kBk;
            if (w < nwork) {
                uint32_t off[3];
                offsets_small<ND, U24>(m, w, off);
                x[u] = load4s(a + off[0], vm.ia, vm.a);
                y[u] = load4s(b + off[1], vm.ib, vm.b);
                oo[u] = off[2];
            }
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const uint32_t w = base + u * kBk;
            if (w < nwork) {
                f4 r;
                r.x = bin<OP>(x[u].x, y[u].x);
                r.y = bin<OP>(x[u].y, y[u].y);
                r.z = bin<OP>(x[u].z, y[u].z);
                r.w = bin<OP>(x[u].w, y[u].w);
                if constexpr (NC_BIN_NT_STORE) __builtin_nontemporal_store(r, (f4 *)(o + oo[u]));
                else *(f4 *)(o + oo[u]) = r;
            }
        }
    }
}

// 64-bit fallback, one element per work item, for outputs that cannot be cut into launches of the
// 32-bit kernels (a single coalesced dim of 2^30 or more elements under a dim that is not merged
// with it): sizes and offsets in int64
struct BigMap {
    int nd;
    int64_t size[NC_HIP_MAX_DIMS];
    int64_t st[3][NC_HIP_MAX_DIMS];
};

template <int OP>
__global__ __launch_bounds__(kB) void k_binary_fwd_big(const float *__restrict__ a, const float *__restrict__ b,
                                                       float *__restrict__ o, BigMap m, int64_t n) {
    const int64_t step = (int64_t)gridDim.x * kB;
    for (int64_t w = (int64_t)blockIdx.x * kB + threadIdx.x; w < n; w += step) {
        int64_t rem = w, oa = 0, ob = 0, oo = 0;
        for (int d = m.nd - 1; d >= 0; d--) {
            const int64_t i = rem % m.size[d];
            rem /= m.size[d];
            oa += i * m.st[0][d];
            ob += i * m.st[1][d];
            oo += i * m.st[2][d];
        }
        o[oo] = bin<OP>(a[oa], b[ob]);
    }
}

struct Prepared {
    int nd;
    int64_t shape[NC_HIP_MAX_DIMS];
    int64_t st[5][NC_HIP_MAX_DIMS];
    int64_t numel;
};

static int prepare(int nd, const int64_t *shape, int nops, const int64_t *const *strides, Prepared &p,
                   const char *who) {
    if (nd < 0 || nd > NC_HIP_MAX_DIMS) return set_error(NC_HIP_ERR_ARG, "%s: ndim %d out of range", who, nd);
    p.numel = 1;
    for (int d = 0; d < nd; d++) {
        if (shape[d] < 0) return set_error(NC_HIP_ERR_ARG, "%s: negative dim", who);
        p.shape[d] = shape[d];
        p.numel *= shape[d];
        for (int o = 0; o < nops; o++) p.st[o][d] = strides[o][d];
    }
    p.nd = p.numel ? coalesce(nd, p.shape, nops, p.st) : 0;
    return NC_HIP_OK;
}

template <int NOPS>
static void make_map(const Prepared &p, int unit, IdxMap<NOPS> &m) {
    m.nd = p.nd;
    for (int d = 0; d < p.nd; d++) {
        const int64_t sz = d == p.nd - 1 ? p.shape[d] / unit : p.shape[d];
        m.size[d] = (uint32_t)sz;
        m.div[d] = IntDiv((uint32_t)sz);
        for (int o = 0; o < NOPS; o++) m.st[o][d] = d == p.nd - 1 ? p.st[o][d] * unit : p.st[o][d];
    }
    for (int d = p.nd; d < NC_HIP_MAX_DIMS; d++) {
        m.size[d] = 1;
        m.div[d] = IntDiv(1);
        for (int o = 0; o < NOPS; o++) m.st[o][d] = 0;
    }
}

static int vec_mode(const float *base, const Prepared &p, int o) {
    const int64_t is = p.st[o][p.nd - 1];
    if (is == 0) return 0;
    if (is != 1) return 2;
    if (!aligned16(base)) return -1;
    for (int d = 0; d < p.nd - 1; d++)
        if (p.st[o][d] % 4) return -1;
    return 1;
}

// Touches one float per 64 bytes of a range so it is cache-resident (L2 / MALL) before a kernel that
// re-reads it many times starts; the loaded values only feed an empty asm statement.
__global__ __launch_bounds__(64) void k_touch(const float *__restrict__ p, int64_t n_lines) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i < n_lines) {
        const float v = p[i * 16];
        asm volatile("" ::"v"(v));
    }
}

// A broadcast operand that occupies a dense memory range much smaller than the output is read by
// every output row that maps to it; warming the range first turns the forward's first touches of it
// from HBM misses into cache hits (a[64,512,1,64], 8 MiB, broadcast into 2^30 outputs: 906 -> 717-745
// us with the forward's launch shape).
static void warm_operand(const float *x, const Prepared &p, int k, hipStream_t st) {
    int64_t hi = 0, distinct = 1;
    for (int d = 0; d < p.nd; d++) {
        if (p.st[k][d] == 0) continue;
        if (p.st[k][d] < 0) return;
        hi += (p.shape[d] - 1) * p.st[k][d];
        distinct *= p.shape[d];
    }
    const int64_t bytes = distinct * 4;
    if (hi + 1 != distinct || distinct * 8 > p.numel || bytes < (1 << 20) || bytes > (128 << 20)) return;
    const int64_t lines = (bytes + 63) / 64;
    hipLaunchKernelGGL(k_touch, dim3((unsigned)((lines + 63) / 64)), dim3(64), 0, st, x, lines);
}

// 0: the 64-bit index kernel; 1: the 32-bit index kernel; 2: the same with 24-bit products
static int small_kind(const Prepared &p, int unit, int64_t nwork) {
    if (p.nd < 1 || p.nd > 4 || nwork >= (int64_t(1) << 31)) return 0;
    bool u24 = true;
    int64_t outer = 1;  // the quotient formed at dim d is below the product of the outer sizes
    for (int d = 0; d < p.nd; d++) {
        const int64_t sz = d == p.nd - 1 ? p.shape[d] / unit : p.shape[d];
        if (sz >= (1 << 24) || (d > 0 && outer > (1 << 24))) u24 = false;
        outer *= sz;
    }
    for (int o = 0; o < 3; o++) {
        int64_t hi = 0;
        for (int d = 0; d < p.nd; d++) {
            const int64_t s = p.st[o][d];
            if (s < 0) return 0;
            hi += (p.shape[d] - 1) * s;
            if ((d == p.nd - 1 ? s * unit : s) >= (1 << 24)) u24 = false;
        }
        if (hi >= (int64_t(1) << 31)) return 0;
    }
    return u24 ? 2 : 1;
}

template <int OP, int ND, bool U24>
static void launch_small(const float *a, const float *b, float *o, const IdxMap<3> &full, SmallModes vm,
                         uint32_t nwork, hipStream_t st) {
    SmallMap<ND> m;
    for (int d = 0; d < ND; d++) {
        m.size[d] = full.size[d];
        m.mul[d] = full.div[d].m;
        m.shift[d] = full.div[d].s;
        for (int k = 0; k < 3; k++) m.st[k][d] = (uint32_t)full.st[k][d];
    }
    constexpr int kU = small_unroll<OP>(), kBk = small_block<OP>();
    const unsigned grid = stream_grid(((int64_t)nwork + kU - 1) / kU, kBk, NC_BIN_GRID_PER_CU);
    hipLaunchKernelGGL((k_binary_fwd_s<OP, ND, U24>), dim3(grid), dim3(kBk), 0, st, a, b, o, m, vm, nwork);
}

template <int OP>
static int launch_fwd(const float *a, const float *b, float *o, const Prepared &p, hipStream_t st) {
    if (p.numel == 0) return NC_HIP_OK;
    if (p.nd == 0) {  // a single element
        IdxMap<3> m;
        Prepared q = p;
        q.nd = 1;
        q.shape[0] = 1;
        q.st[0][0] = q.st[1][0] = q.st[2][0] = 0;
        make_map<3>(q, 1, m);
        hipLaunchKernelGGL((k_binary_fwd<OP, false>), dim3(1), dim3(kBF), 0, st, a, b, o, m, VecModes{}, 1u);
        return check_launch("nc_hip_binary_fwd");
    }
    const int inner = p.nd - 1;
    int ma = vec_mode(a, p, 0), mb = vec_mode(b, p, 1);
    const bool vec = p.st[2][inner] == 1 && p.shape[inner] % 4 == 0 && vec_mode(o, p, 2) == 1 && ma >= 0 && mb >= 0;
    const int unit = vec ? 4 : 1;
    const int64_t nwork = p.numel / unit;
    // Outputs past the 32-bit kernels' reach (2^31 work items, or an operand offset of 2^31 elements
    // or more) are cut along the outermost coalesced dim into runs of at most 2^30 outputs, each a
    // launch of its own with the operand bases advanced: the full [256,512,512,64] broadcast runs as
    // the same 2^30-output launches as its chunks.
    int64_t hi = 0;
    for (int k = 0; k < 3; k++) {
        int64_t h = 0;
        for (int d = 0; d < p.nd; d++) h += (p.shape[d] - 1) * (p.st[k][d] < 0 ? -p.st[k][d] : p.st[k][d]);
        hi = std::max(hi, h);
    }
    if (nwork >= (int64_t(1) << 31) || hi >= (int64_t(1) << 31)) {
        const int64_t S0 = p.shape[0], per = p.numel / S0;  // outputs per index of the outer dim
        int64_t run = (int64_t(1) << 30) / per;
        for (int k = 0; k < 3 && run > 0; k++) {  // keep every operand's offsets of a run below 2^31
            const int64_t s0 = p.st[k][0] < 0 ? -p.st[k][0] : p.st[k][0];
            int64_t rest = 0;
            for (int d = 1; d < p.nd; d++) rest += (p.shape[d] - 1) * (p.st[k][d] < 0 ? -p.st[k][d] : p.st[k][d]);
            if (s0 > 0) run = std::min(run, ((int64_t(1) << 31) - 1 - rest) / s0 + 1);
            if (rest >= (int64_t(1) << 31)) run = 0;
        }
        if (p.nd == 1) run -= run % 4;  // keep 16-byte alignment of every piece but the last
        if (run >= 1 && run < S0) {
            for (int64_t r0 = 0; r0 < S0; r0 += run) {
                Prepared q = p;
                q.shape[0] = std::min(run, S0 - r0);
                q.numel = q.shape[0] * per;
                const int rc = launch_fwd<OP>(a + r0 * p.st[0][0], b + r0 * p.st[1][0], o + r0 * p.st[2][0], q, st);
                if (rc != NC_HIP_OK) return rc;
            }
            return NC_HIP_OK;
        }
    }
    if (nwork >= (int64_t)UINT32_MAX) {
        BigMap m{};
        m.nd = p.nd;
        for (int d = 0; d < p.nd; d++) {
            m.size[d] = p.shape[d];
            for (int k = 0; k < 3; k++) m.st[k][d] = p.st[k][d];
        }
        hipLaunchKernelGGL(k_binary_fwd_big<OP>, dim3(stream_grid(p.numel, kB)), dim3(kB), 0, st, a, b, o, m,
                           p.numel);
        return check_launch("nc_hip_binary_fwd");
    }
    IdxMap<3> m;
    make_map<3>(p, unit, m);
    if (NC_BIN_WARM) {
        warm_operand(a, p, 0, st);
        warm_operand(b, p, 1, st);
    }
    const unsigned grid = stream_grid((nwork + kBU - 1) / kBU, kBF, NC_BIN_GRID_PER_CU);
    const int kind = vec && NC_BIN_SMALL_INDEX ? small_kind(p, unit, nwork) : 0;
    if (kind) {
        // an operand with no broadcast dim is read once: non-temporal loads
        auto once = [&](int k) {
            for (int d = 0; d < p.nd; d++)
                if (p.st[k][d] == 0 && p.shape[d] > 1) return false;
            return true;
        };
        SmallModes vm{ma == 1 && once(0) ? 3 : ma, mb == 1 && once(1) ? 3 : mb, (uint32_t)p.st[0][inner],
                      (uint32_t)p.st[1][inner]};
        switch (p.nd * 2 + (kind == 2)) {
#define NC_BIN_SMALL(ND)                                                                                        \
    case 2 * ND: launch_small<OP, ND, false>(a, b, o, m, vm, (uint32_t)nwork, st); break;                 \
    case 2 * ND + 1: launch_small<OP, ND, true>(a, b, o, m, vm, (uint32_t)nwork, st); break;
            NC_BIN_SMALL(1)
            NC_BIN_SMALL(2)
            NC_BIN_SMALL(3)
            NC_BIN_SMALL(4)
#undef NC_BIN_SMALL
        }
    } else if (vec) {
        VecModes vm{ma, mb, p.st[0][inner], p.st[1][inner]};
        hipLaunchKernelGGL((k_binary_fwd<OP, true>), dim3(grid), dim3(kBF), 0, st, a, b, o, m, vm, (uint32_t)nwork);
    } else {
        hipLaunchKernelGGL((k_binary_fwd<OP, false>), dim3(grid), dim3(kBF), 0, st, a, b, o, m, VecModes{},
                           (uint32_t)nwork);
    }
    return check_launch("nc_hip_binary_fwd");
}

// ------------------------------------------------------------------------------------------------
// gradients
// ------------------------------------------------------------------------------------------------
// fp32 term with the reference's association (unreduced grads: bit-identical)
// mode: 0 alpha*g, 1 g*p1, 2 g/p1, 3 -(g*p1)/(p2*p2)
template <int MODE>
__device__ __forceinline__ float grad_f(float gi, float g, float p1, float p2, float alpha) {
    if constexpr (MODE == 0) return fma_(alpha, g, gi);  // axpy_f32 (same-shape add/sub, ops_elementwise.c:162-164)
    else if constexpr (MODE == 1) return gi + g * p1;
    else if constexpr (MODE == 2) return gi + g / p1;
    else return gi - (g * p1) / (p2 * p2);
}

// fp64 term for reduced grads
template <int MODE>
__device__ __forceinline__ double grad_d(double g, double p1, double p2, double alpha) {
    if constexpr (MODE == 0) return alpha * g;
    else if constexpr (MODE == 1) return g * p1;
    else if constexpr (MODE == 2) return g / p1;
    else return -(g * p1) / (p2 * p2);
}

// operand order in the maps: 0 g, 1 p1, 2 p2, 3 gx
template <int MODE, bool ACC>
__global__ __launch_bounds__(kB) void k_grad_elementwise(const float *__restrict__ g, const float *__restrict__ p1,
                                                         const float *__restrict__ p2, float *__restrict__ gx,
                                                         IdxMap<4> m, uint32_t nwork, float alpha) {
    const uint32_t step = gridDim.x * kB;
    for (uint32_t w = blockIdx.x * kB + threadIdx.x; w < nwork; w += step) {
        int64_t off[4];
        offsets<4>(m, w, off);
        const float v1 = MODE == 1 || MODE == 2 || MODE == 3 ? p1[off[1]] : 0.0f;
        const float v2 = MODE == 3 ? p2[off[2]] : 0.0f;
        const float old = ACC ? gx[off[3]] : 0.0f;
        gx[off[3]] = grad_f<MODE>(old, g[off[0]], v1, v2, alpha);
    }
}

// The same for contiguous, 16-byte aligned operands of one shape (residual and elementwise-product
// backward): one float4 of each stream per lane, non-temporal, a grid over the whole range.
template <int MODE, bool ACC>
__global__ __launch_bounds__(64) void k_grad_elementwise4(const f4 *__restrict__ g, const f4 *__restrict__ p1,
                                                          const f4 *__restrict__ p2, f4 *__restrict__ gx, int64_t n4,
                                                          float alpha) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i >= n4) return;
    const f4 z = f4{0.f, 0.f, 0.f, 0.f};
    const f4 gg = __builtin_nontemporal_load(g + i);
    const f4 a = MODE == 1 || MODE == 2 || MODE == 3 ? __builtin_nontemporal_load(p1 + i) : z;
    const f4 b = MODE == 3 ? __builtin_nontemporal_load(p2 + i) : z;
    const f4 o = ACC ? __builtin_nontemporal_load(gx + i) : z;
    f4 r;
    r.x = grad_f<MODE>(o.x, gg.x, a.x, b.x, alpha);
    r.y = grad_f<MODE>(o.y, gg.y, a.y, b.y, alpha);
    r.z = grad_f<MODE>(o.z, gg.z, a.z, b.z, alpha);
    r.w = grad_f<MODE>(o.w, gg.w, a.w, b.w, alpha);
    __builtin_nontemporal_store(r, gx + i);
}

// Reduced grads.  The coalesced dims split into kept dims (gx stride != 0) and reduced dims.
struct RedPlan {
    IdxMap<4> kept;      // over the M kept indices (gx offsets in operand 3)
    IdxMap<3> red;       // over the K reduced indices (g, p1, p2 offsets)
    uint32_t M, K;
    uint32_t chunk;      // reduced indices per partial
    uint32_t P;          // partials per kept index
    int inner_kept;      // 1: lanes <-> kept indices (column mode), 0: lanes <-> reduced (row mode)
};

// column mode: one lane per kept index, sequential over a chunk of reduced indices (odometer)
template <int MODE>
__global__ __launch_bounds__(kB) void k_grad_reduce_col(const float *__restrict__ g, const float *__restrict__ p1,
                                                        const float *__restrict__ p2, RedPlan pl, double alpha,
                                                        double *__restrict__ part) {
    const uint64_t total = (uint64_t)pl.M * pl.P;
    for (uint64_t item = (uint64_t)blockIdx.x * kB + threadIdx.x; item < total; item += (uint64_t)gridDim.x * kB) {
    const uint32_t mi = (uint32_t)(item % pl.M);
    const uint32_t p = (uint32_t)(item / pl.M);
    int64_t ko[4];
    offsets<4>(pl.kept, mi, ko);
    const uint32_t k0 = p * pl.chunk;
    const uint32_t k1 = min(pl.K, k0 + pl.chunk);
    // starting reduced coordinates
    uint32_t idx[NC_HIP_MAX_DIMS];
    int64_t ro[3] = {0, 0, 0};
    {
        uint32_t w = k0;
#pragma unroll
        for (int d = NC_HIP_MAX_DIMS - 1; d >= 0; d--) {
            if (d < pl.red.nd) {
                const uint32_t q = pl.red.div[d].div(w);
                idx[d] = w - q * pl.red.size[d];
                w = q;
#pragma unroll
                for (int o = 0; o < 3; o++) ro[o] += (int64_t)idx[d] * pl.red.st[o][d];
            }
        }
    }
    const int inner = pl.red.nd - 1;
    const int64_t s0 = pl.red.st[0][inner], s1 = pl.red.st[1][inner], s2 = pl.red.st[2][inner];
    const uint32_t n_in = pl.red.size[inner];
    double acc = 0.0;
    uint32_t k = k0;
    while (k < k1) {
        // run along the innermost reduced dim without carries
        const uint32_t run = min(k1 - k, n_in - idx[inner]);
        const float *pg = g + ko[0] + ro[0];
        const float *q1 = p1 + ko[1] + ro[1];
        const float *q2 = p2 + ko[2] + ro[2];
        for (uint32_t r = 0; r < run; r++) {
            const double v1 = (MODE == 1 || MODE == 2 || MODE == 3) ? (double)q1[r * s1] : 0.0;
            const double v2 = MODE == 3 ? (double)q2[r * s2] : 0.0;
            acc += grad_d<MODE>((double)pg[r * s0], v1, v2, alpha);
        }
        k += run;
        if (k >= k1) break;
        // carry into the outer reduced dims
        ro[0] += (int64_t)run * s0;
        ro[1] += (int64_t)run * s1;
        ro[2] += (int64_t)run * s2;
        idx[inner] += run;
        for (int d = inner; d >= 0; d--) {
            if (idx[d] < pl.red.size[d]) break;
            ro[0] -= (int64_t)idx[d] * pl.red.st[0][d];
            ro[1] -= (int64_t)idx[d] * pl.red.st[1][d];
            ro[2] -= (int64_t)idx[d] * pl.red.st[2][d];
            idx[d] = 0;
            if (d > 0) {
                idx[d - 1]++;
                ro[0] += pl.red.st[0][d - 1];
                ro[1] += pl.red.st[1][d - 1];
                ro[2] += pl.red.st[2][d - 1];
            }
        }
    }
    part[(size_t)p * pl.M + mi] = acc;
    }
}

// row mode: one block per (kept index, chunk of reduced indices); lanes stride over the chunk
template <int MODE>
__global__ __launch_bounds__(kB) void k_grad_reduce_row(const float *__restrict__ g, const float *__restrict__ p1,
                                                        const float *__restrict__ p2, RedPlan pl, double alpha,
                                                        double *__restrict__ part) {
    __shared__ double sh[kB / kWave];
    const uint64_t total = (uint64_t)pl.M * pl.P;
    for (uint64_t item = blockIdx.x; item < total; item += gridDim.x) {  // block-uniform loop
        const uint32_t mi = (uint32_t)(item % pl.M);
        const uint32_t p = (uint32_t)(item / pl.M);
        int64_t ko[4];
        offsets<4>(pl.kept, mi, ko);
        const uint32_t k0 = p * pl.chunk;
        const uint32_t k1 = min(pl.K, k0 + pl.chunk);
        double acc = 0.0;
        for (uint32_t k = k0 + threadIdx.x; k < k1; k += kB) {
            int64_t ro[3];
            offsets<3>(pl.red, k, ro);
            const double v1 = (MODE == 1 || MODE == 2 || MODE == 3) ? (double)p1[ko[1] + ro[1]] : 0.0;
            const double v2 = MODE == 3 ? (double)p2[ko[2] + ro[2]] : 0.0;
            acc += grad_d<MODE>((double)g[ko[0] + ro[0]], v1, v2, alpha);
        }
        acc = wave_sum(acc);
        if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = acc;
        __syncthreads();
        if (threadIdx.x == 0) {
            double t = 0.0;
#pragma unroll
            for (int i = 0; i < kB / kWave; i++) t += sh[i];
            part[(size_t)p * pl.M + mi] = t;
        }
        __syncthreads();
    }
}

// gx[kept m] (+)= sum over partials, in partial order
template <bool ACC>
__global__ __launch_bounds__(kB) void k_grad_finalize(const double *__restrict__ part, float *__restrict__ gx,
                                                      IdxMap<4> kept, uint32_t M, uint32_t P) {
    const uint32_t mi = blockIdx.x * kB + threadIdx.x;
    if (mi >= M) return;
    int64_t ko[4];
    offsets<4>(kept, mi, ko);
    double t = ACC ? (double)gx[ko[3]] : 0.0;
    // the partials in order, their loads issued kU at a time (49 partials: 9.5 -> 3 us)
    constexpr uint32_t kU = 8;
    uint32_t p = 0;
    for (; p + kU <= P; p += kU) {
        double v[kU];
#pragma unroll
        for (uint32_t u = 0; u < kU; u++) v[u] = part[(size_t)(p + u) * M + mi];
#pragma unroll
        for (uint32_t u = 0; u < kU; u++) t += v[u];
    }
    for (; p < P; p++) t += part[(size_t)p * M + mi];
    gx[ko[3]] = (float)t;
}

static int grad_mode(int op, int which) {
    if (op == NC_HIP_BIN_ADD || op == NC_HIP_BIN_SUB) return 0;
    if (op == NC_HIP_BIN_MUL || which == 0) return op == NC_HIP_BIN_MUL ? 1 : 2;
    return 3;
}

// Builds the reduction plan; returns false when nothing is reduced.
static bool plan_reduce(const Prepared &p, RedPlan &pl, size_t *ws_need) {
    Prepared kp{}, rp{};
    kp.nd = rp.nd = 0;
    uint64_t M = 1, K = 1;
    for (int d = 0; d < p.nd; d++) {
        if (p.st[3][d] == 0) {
            rp.shape[rp.nd] = p.shape[d];
            for (int o = 0; o < 3; o++) rp.st[o][rp.nd] = p.st[o][d];
            rp.nd++;
            K *= (uint64_t)p.shape[d];
        } else {
            kp.shape[kp.nd] = p.shape[d];
            for (int o = 0; o < 4; o++) kp.st[o][kp.nd] = p.st[o][d];
            kp.nd++;
            M *= (uint64_t)p.shape[d];
        }
    }
    if (rp.nd == 0) return false;
    if (kp.nd == 0) {  // full reduction: one kept index
        kp.nd = 1;
        kp.shape[0] = 1;
        for (int o = 0; o < 4; o++) kp.st[o][0] = 0;
    }
    make_map<4>(kp, 1, pl.kept);
    make_map<3>(rp, 1, pl.red);
    pl.M = (uint32_t)M;
    pl.K = (uint32_t)K;
    pl.inner_kept = p.nd > 0 && p.st[3][p.nd - 1] != 0;
    const uint64_t target = (uint64_t)kPlanCUs * 2048;  // lanes to keep every CU busy (shape-only plan)
    if (pl.inner_kept) {
        uint64_t P = (target + M - 1) / M;
        uint64_t maxP = (K + 63) / 64;  // at least 64 terms per lane
        if (P > maxP) P = maxP;
        if (P < 1) P = 1;
        pl.chunk = (uint32_t)((K + P - 1) / P);
        pl.P = (uint32_t)((K + pl.chunk - 1) / pl.chunk);
    } else {
        uint64_t blocks_target = (uint64_t)kPlanCUs * 8;
        uint64_t P = (blocks_target + M - 1) / M;
        uint64_t maxP = (K + 4 * kB - 1) / (4 * kB);  // at least 4 terms per lane
        if (P > maxP) P = maxP;
        if (P < 1) P = 1;
        pl.chunk = (uint32_t)((K + P - 1) / P);
        pl.P = (uint32_t)((K + pl.chunk - 1) / pl.chunk);
    }
    *ws_need = (size_t)pl.P * pl.M * sizeof(double);
    return true;
}

template <int MODE>
static int launch_grad(const float *g, const float *p1, const float *p2, float *gx, const Prepared &p, float alpha,
                       int acc, void *ws, size_t ws_bytes, hipStream_t st) {
    if (p.numel == 0) return NC_HIP_OK;
    RedPlan pl;
    size_t need = 0;
    if (!plan_reduce(p, pl, &need)) {
        Prepared q = p;
        if (q.nd == 0) {
            q.nd = 1;
            q.shape[0] = 1;
            for (int o = 0; o < 4; o++) q.st[o][0] = 0;
        }
        constexpr bool R1 = MODE == 1 || MODE == 2 || MODE == 3, R2 = MODE == 3;
        if (q.nd == 1 && q.numel % 4 == 0 && q.st[0][0] == 1 && q.st[3][0] == 1 && (!R1 || q.st[1][0] == 1) &&
            (!R2 || q.st[2][0] == 1) && aligned16(g) && aligned16(gx) && (!R1 || aligned16(p1)) &&
            (!R2 || aligned16(p2))) {
            const int64_t n4 = q.numel / 4;
            const dim3 grid4((unsigned)((n4 + 63) / 64));
            if (acc)
                hipLaunchKernelGGL((k_grad_elementwise4<MODE, true>), grid4, dim3(64), 0, st, (const f4 *)g,
                                   (const f4 *)p1, (const f4 *)p2, (f4 *)gx, n4, alpha);
            else
                hipLaunchKernelGGL((k_grad_elementwise4<MODE, false>), grid4, dim3(64), 0, st, (const f4 *)g,
                                   (const f4 *)p1, (const f4 *)p2, (f4 *)gx, n4, alpha);
            return check_launch("nc_hip_binary_bwd");
        }
        IdxMap<4> m;
        make_map<4>(q, 1, m);
        if (p.numel >= (int64_t)UINT32_MAX) return set_error(NC_HIP_ERR_ARG, "grad: 2^32 or more elements");
        const unsigned grid = stream_grid(p.numel, kB, 16);
        if (acc)
            hipLaunchKernelGGL((k_grad_elementwise<MODE, true>), dim3(grid), dim3(kB), 0, st, g, p1, p2, gx, m,
                               (uint32_t)p.numel, alpha);
        else
            hipLaunchKernelGGL((k_grad_elementwise<MODE, false>), dim3(grid), dim3(kB), 0, st, g, p1, p2, gx, m,
                               (uint32_t)p.numel, alpha);
        return check_launch("nc_hip_binary_bwd");
    }
    if (p.numel >= (int64_t)UINT32_MAX)
        return set_error(NC_HIP_ERR_ARG, "grad: sum-to-shape over 2^32 or more elements is not supported");
    if (ws_bytes < need || (need && !ws))
        return set_error(NC_HIP_ERR_WORKSPACE, "grad: workspace of %zu bytes needed, %zu given", need, ws_bytes);
    double *part = (double *)ws;
    const uint64_t items = (uint64_t)pl.M * pl.P;
    if (pl.inner_kept) {
        const uint64_t blocks = (items + kB - 1) / kB;
        const unsigned grid = (unsigned)(blocks < 1048576 ? blocks : 1048576);
        hipLaunchKernelGGL(k_grad_reduce_col<MODE>, dim3(grid), dim3(kB), 0, st, g, p1, p2, pl, (double)alpha, part);
    } else {
        const unsigned grid = (unsigned)(items < 1048576 ? items : 1048576);
        hipLaunchKernelGGL(k_grad_reduce_row<MODE>, dim3(grid), dim3(kB), 0, st, g, p1, p2, pl, (double)alpha, part);
    }
    const unsigned fg = (pl.M + kB - 1) / kB;
    if (acc)
        hipLaunchKernelGGL(k_grad_finalize<true>, dim3(fg), dim3(kB), 0, st, part, gx, pl.kept, pl.M, pl.P);
    else
        hipLaunchKernelGGL(k_grad_finalize<false>, dim3(fg), dim3(kB), 0, st, part, gx, pl.kept, pl.M, pl.P);
    return check_launch("nc_hip_binary_bwd");
}

static int prepare_grad(int op, int which, int nd, const int64_t *shape, const int64_t *sg, const int64_t *sa,
                        const int64_t *sb, const int64_t *sgx, Prepared &p, int &mode, float &alpha,
                        bool &p1_is_a) {
    mode = grad_mode(op, which);
    alpha = (op == NC_HIP_BIN_SUB && which == 1) ? -1.0f : 1.0f;
    // p1 = other operand (mul), b (div wrt a), a (div wrt b); p2 = b (div wrt b)
    p1_is_a = (op == NC_HIP_BIN_MUL && which == 1) || (op == NC_HIP_BIN_DIV && which == 1);
    const int64_t *s1 = p1_is_a ? sa : sb;
    const int64_t zeros[NC_HIP_MAX_DIMS] = {0, 0, 0, 0, 0, 0};
    if (mode == 0) s1 = zeros;
    const int64_t *s2 = mode == 3 ? sb : zeros;
    const int64_t *strides[4] = {sg, s1, s2, sgx};
    return prepare(nd, shape, 4, strides, p, "nc_hip_binary_bwd");
}

// ------------------------------------------------------------------------------------------------
// Fused backward of both operands (one pass over g) for the pattern
//     g[P..., H, W] (contiguous),  a[P..., 1, W] (broadcast over H),  b[H, W] (broadcast over P...)
// i.e. grad_a = sum over H, grad_b = sum over the plane dims.
//   * A plane of H*W/4 float4 is cut into NBAND row bands of 512*T float4 (T <= NC_B2_TMAX); a
//     512-lane workgroup owns one band of a range of planes.  Lane t holds float4 q = t + 512 k
//     (k < T) of the band, all in column group w4 = t mod W4 (W4 = W/4 divides 64).
//   * g: the T loads of the next plane (and, for mul and div, a's row of it) are issued before the
//     current plane is summed.
//   * Launch shape: when grad_a is written, T = 8 where the plane allows it, with one workgroup
//     per CU (256 VGPRs per lane): twice the bytes per lane per plane of T = 4 at two workgroups
//     per CU, so the per-plane grad_a exchange (shuffles, LDS slots, group sums, partial stores)
//     is paid per twice the data (2^30-output backward: 775 -> 732 us).  grad_b alone has no
//     exchange and runs T <= 4 with one workgroup per CU.
//   * grad_b accumulates in fp64 registers (T x 4 per lane) over the workgroup's planes and is written
//     once as a partial, combined by k_bwd2_gb_combine in plane-range order.
//   * b (mul) or its fp32 reciprocal (div) stays in registers.  Each term is an fp32 product, as in
//     the unreduced gradient (g*b, g*a; g*(1/b) is within 1 ulp of g/b), and the sums run in fp64.
//     A wave whose b includes a nonzero subnormal (1/b overflows there) divides g / b instead.
//   * grad_a: per plane, lanes sharing w4 are reduced by wave shuffles; the 8 wave partials of a
//     group of NB = 64 / W4 planes wait in LDS, and after one barrier per group a lane per (plane,
//     column) adds them in wave order.  With one band that sum completes grad_a; with several it is an
//     fp64 partial that k_bwd2_ga_combine adds up in band order.
// MODE: 0 add/sub, 1 mul, 3 div.
// ------------------------------------------------------------------------------------------------
#ifndef NC_B2_TMAX
#define NC_B2_TMAX 8  // T when grad_a is written
#endif
#ifndef NC_B2_GB_TMAX
#define NC_B2_GB_TMAX 4  // T for grad_b alone
#endif
constexpr int kB2 = 512;
constexpr int kB2Waves = kB2 / kWave;
constexpr int kB2MaxBand = 16;  // bands per plane: planes up to 16 * 512 * T float4
constexpr int kB2GroupDoubles = kB2Waves * 4 * 64;
// Groups of grad_a held in LDS between stores, sized so that the slot sets and res fill the CU's
// 160 KiB of LDS at the launch's workgroups per CU.  A drain of res is a burst of stores that the
// next plane loads wait behind (one in-order memory counter): at one drain per 64 planes the
// 2^30-output backward took 728 us, with none before the end 648 us, so the plan gives each
// workgroup no more planes than res holds where the problem allows.
constexpr uint32_t b2_res_groups(int64_t T) { return T >= 8 ? 64 : 24; }

struct Bwd2Plan {
    uint32_t P, H, W4, T, nband;
    uint32_t ranges, planes_per_block;
    IdxMap<1> amap;  // element offset of a[p, 0, 0] over the plane dims
};

// OUT selects the gradients written: 1 grad_a, 2 grad_b, 3 both.
// two resident workgroups per CU (4 waves per SIMD): at most 128 VGPRs
template <int MODE, bool ACC, int T, int OUT>
__global__ __launch_bounds__(kB2, T >= 8 ? 2 : 4) void k_bcast_bwd2(const float *__restrict__ g, const float *__restrict__ a,
                                                    const float *__restrict__ b, float *__restrict__ ga,
                                                    double *__restrict__ ga_part, double *__restrict__ gb_part,
                                                    Bwd2Plan pl, double alpha_b) {
    constexpr uint32_t band4 = kB2 * T;  // float4 per band
    __shared__ double sh[2][kB2GroupDoubles];  // two group slot sets, each [NB][8 waves][W4][4]
    constexpr uint32_t kB2ResGroups = b2_res_groups(T);
    __shared__ double res[kB2ResGroups * 4 * 64];  // grad_a of the last kB2ResGroups groups, [plane][W]
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    const uint32_t W4 = pl.W4, nband = pl.nband;
    const uint32_t NB = 64 / W4;
    const uint32_t w4 = tid % W4;
    const uint32_t band = blockIdx.x % nband, range = blockIdx.x / nband;
    const uint32_t plane4 = band4 * nband;
    const uint32_t p0 = range * pl.planes_per_block;
    const uint32_t p1 = min(pl.P, p0 + pl.planes_per_block);  // the launch has p0 < P for every workgroup
    const uint32_t qb = band * band4 + tid;                    // this lane's first float4 in a plane
    constexpr bool WA = OUT & 1, WB = OUT & 2;
    f4 bv[T];
    bool tiny = false;  // a nonzero subnormal b, whose reciprocal overflows
#pragma unroll
    for (int k = 0; k < T; k++) {
        bv[k] = f4{1.f, 1.f, 1.f, 1.f};
        if constexpr (WA && MODE != 0) bv[k] = ((const f4 *)b)[qb + kB2 * k];
        if constexpr (WA && MODE == 3) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float m = __builtin_fabsf(bv[k][c]);
                tiny |= m != 0.0f && m < 0x1p-126f;
            }
            bv[k] = f4{1.0f / bv[k].x, 1.0f / bv[k].y, 1.0f / bv[k].z, 1.0f / bv[k].w};
        }
    }
    // wave-uniform: a wave holding such a b divides (g / b, reloading b) instead of multiplying by
    // the reciprocal, so grad_a stays finite where the reference's g / b is
    const bool exact_div = WA && MODE == 3 && __ballot(tiny) != 0;
    double accb[T][4];
#pragma unroll
    for (int k = 0; k < T; k++) accb[k][0] = accb[k][1] = accb[k][2] = accb[k][3] = 0.0;
    f4 cur[T];
    {
        const f4 *gp = (const f4 *)g + (size_t)p0 * plane4 + qb;
#pragma unroll
        for (int k = 0; k < T; k++) cur[k] = __builtin_nontemporal_load(gp + kB2 * k);
    }
    // a[p, this lane's 4 columns] (grad_b terms of mul and div), loaded one plane ahead with g
    constexpr bool RA = WB && (MODE == 1 || MODE == 3);
    auto load_a = [&](uint32_t p) {
        int64_t off[1];
        offsets<1>(pl.amap, p, off);
        return *(const f4 *)(a + off[0] + 4 * w4);
    };
    f4 av = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (RA) av = load_a(p0);
    // grad_a of the nb planes of group gi: lane -> (plane j, column col, component c), the 8 wave
    // partials added in wave order, into the group's slot of res
    const uint32_t WE = 4 * W4;  // grad_a elements per plane
    auto flush = [&](uint32_t gi, uint32_t nb) {
        const double *set = sh[gi & 1];
        double *dst = res + (gi % kB2ResGroups) * NB * WE;
        for (uint32_t idx = tid; idx < WE * nb; idx += kB2) {
            const uint32_t c = idx % 4, col = (idx / 4) % W4, j = idx / WE;
            double t = 0.0;
#pragma unroll
            for (int w = 0; w < kB2Waves; w++) t += set[((j * kB2Waves + w) * W4 + col) * 4 + c];
            dst[j * WE + 4 * col + c] = t;
        }
    };
    // res -> grad_a (one band) or this band's fp64 partials, for the np planes from `first` (the
    // first plane of a res-aligned run of groups).  Stores are few and bunched: a store waits in the
    // same in-order counter as the plane loads, so each one issued inside the plane loop would make
    // the next wait for data wait for it too.
    auto drain = [&](uint32_t g0, uint32_t np) {
        const uint32_t first = p0 + g0 * NB;
        const double *src = res + (g0 % kB2ResGroups) * NB * WE;
        for (uint32_t idx = tid; idx < WE * np; idx += kB2) {
            const uint32_t pl_ = first + idx / WE, e = idx % WE;
            const double t = src[idx];
            if (nband == 1) {
                const size_t ge = (size_t)pl_ * WE + e;
                ga[ge] = (float)((ACC ? (double)ga[ge] : 0.0) + t);
            } else {
                ga_part[((size_t)pl_ * nband + band) * WE + e] = t;
            }
        }
    };
    uint32_t gi = 0, dg = 0;  // dg: the first group not yet drained
    for (uint32_t pg = p0; pg < p1; pg += NB, gi++) {
        const uint32_t nb = min(NB, p1 - pg);
        for (uint32_t j = 0; j < nb; j++) {
            const uint32_t p = pg + j;
            // next plane's loads first (the last plane loads itself again: in bounds, unused)
            f4 nxt[T];
            {
                const f4 *gn = (const f4 *)g + (size_t)min(p + 1, p1 - 1) * plane4 + qb;
#pragma unroll
                for (int k = 0; k < T; k++) nxt[k] = __builtin_nontemporal_load(gn + kB2 * k);
            }
            f4 avn = av;
            if constexpr (RA) avn = load_a(min(p + 1, p1 - 1));
            if constexpr (WA) {
                if (j == 0 && gi > 0) {
                    lds_barrier();  // every wave has written the previous group's slots
                    flush(gi - 1, NB);
                    if (gi % kB2ResGroups == 0) {  // res holds groups dg = gi - kB2ResGroups .. gi - 1
                        lds_barrier();
                        drain(dg, (gi - dg) * NB);
                        dg = gi;
                    }
                }
            }
            // one component at a time, so that only T grad_a terms are live: terms are the fp32
            // products the unreduced gradient holds, summed in fp64 (grad_a: g for add and sub, g*b
            // for mul, g*(1/b) for div, added as a pairwise tree over the lane's T float4; grad_b
            // before its per-column factor: g for add and sub, g*a for mul and div)
            double sa[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                double ta[T];
#pragma unroll
                for (int k = 0; k < T; k++) {
                    const float gg = cur[k][c];
                    if constexpr (WA) {
                        float t = gg;
                        if constexpr (MODE == 1) t = gg * bv[k][c];
                        if constexpr (MODE == 3)
                            t = exact_div ? gg / ((const f4 *)b)[qb + kB2 * k][c] : gg * bv[k][c];
                        ta[k] = (double)t;
                    }
                    if constexpr (WB) accb[k][c] += (double)((MODE == 1 || MODE == 3) ? gg * av[c] : gg);
                }
                sa[c] = 0.0;
                if constexpr (WA) {
#pragma unroll
                    for (int h = T / 2; h >= 1; h /= 2) {
#pragma unroll
                        for (int k = 0; k < h; k++) ta[k] += ta[k + h];
                    }
                    sa[c] = ta[0];
                }
            }
#pragma unroll
            for (int k = 0; k < T; k++) cur[k] = nxt[k];
            av = avn;
            if constexpr (!WA) continue;
            // lanes sharing w4 inside the wave; the wave's partial goes to LDS slot (j, wv)
            for (uint32_t o = W4; o < (uint32_t)kWave; o <<= 1) {
#pragma unroll
                for (int c = 0; c < 4; c++) sa[c] += __shfl_xor(sa[c], (int)o, kWave);
            }
            if ((uint32_t)lane < W4) {
                double *d = sh[gi & 1] + ((j * kB2Waves + wv) * W4 + lane) * 4;
#pragma unroll
                for (int c = 0; c < 4; c++) d[c] = sa[c];
            }
        }
    }
    if constexpr (WA) {
        // the last group and the rest of res.  Slot sets and res slots are rewritten only after a
        // barrier that every wave reaches after it has finished reading them.
        lds_barrier();
        const uint32_t last = gi - 1;
        flush(last, p1 - (p0 + last * NB));
        lds_barrier();
        drain(dg, p1 - (p0 + dg * NB));
    }
    if constexpr (WB) {
        double *out = gb_part + (size_t)range * plane4 * 4;
#pragma unroll
        for (int k = 0; k < T; k++) {
            const uint32_t q = qb + kB2 * k;
#pragma unroll
            for (int c = 0; c < 4; c++) out[4 * q + c] = accb[k][c] * alpha_b;
        }
    }
}

// grad_a[e] (+)= sum over bands of part[p][band][w] (e = p * W + w), bands in order
template <bool ACC>
__global__ __launch_bounds__(kB) void k_bwd2_ga_combine(const double *__restrict__ part, float *__restrict__ ga,
                                                        uint32_t n, uint32_t W, IntDiv divW, uint32_t nband) {
    const uint32_t step = gridDim.x * kB;
    for (uint32_t e = blockIdx.x * kB + threadIdx.x; e < n; e += step) {
        const uint32_t p = divW.div(e), w = e - p * W;
        const double *src = part + (size_t)p * nband * W + w;
        double t = 0.0;
        for (uint32_t k = 0; k < nband; k++) t += src[(size_t)k * W];
        ga[e] = (float)((ACC ? (double)ga[e] : 0.0) + t);
    }
}

// grad_b[e] (+)= factor(e) * sum over plane ranges of part[r][e], ranges in order (64 x 16 lanes)
template <int MODE, bool ACC>
__global__ __launch_bounds__(1024) void k_bwd2_gb_combine(const double *__restrict__ part, const float *__restrict__ b,
                                                          float *__restrict__ gb, uint32_t n, uint32_t nparts) {
    __shared__ double shc[16][64];
    const int x = threadIdx.x % 64, y = threadIdx.x / 64;
    const uint32_t e = blockIdx.x * 64 + x;
    double t = 0.0;
    if (e < n) {
#pragma unroll 8
        for (uint32_t q = y; q < nparts; q += 16) t += part[(size_t)q * n + e];
    }
    shc[y][x] = t;
    __syncthreads();
    if (y == 0 && e < n) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < 16; k++) s += shc[k][x];
        if constexpr (MODE == 3) {  // d(a/b)/db = -(g a) / b^2: the b factor is the same for every term
            const double bv = (double)b[e];
            s = -s / (bv * bv);
        }
        gb[e] = (float)((ACC ? (double)gb[e] : 0.0) + s);
    }
}

// Returns true (and the plan) when the fused kernel applies to the prepared operand strides
// (order: g, a, b, ga, gb).
// out: the gradients written (1 grad_a, 2 grad_b, 3 both).  The workspace of a plan for 3 covers the
// plans for 1 and 2 of the same problem (the same or fewer plane ranges, the same grad_a bands).
static bool plan_bwd2(const Prepared &p, const float *g, const float *a, const float *b, const float *ga,
                      const float *gb, Bwd2Plan &pl, int out) {
    const int64_t tmax = out == 2 ? NC_B2_GB_TMAX : NC_B2_TMAX;
    if (p.nd < 3 || p.numel >= (int64_t)UINT32_MAX) return false;
    const int h = p.nd - 2, w = p.nd - 1;
    const int64_t H = p.shape[h], W = p.shape[w];
    if (W % 4 || 64 % (W / 4) || (H * (W / 4)) % kB2) return false;
    int64_t T = H * (W / 4) / kB2, nband = 1;  // float4 per lane per plane
    if (T & (T - 1)) return false;
    while (T > tmax) {
        T /= 2;
        nband *= 2;
    }
    if (nband > kB2MaxBand) return false;
    // g contiguous; a: stride 0 over H, 1 over W; b: [H, W] contiguous, 0 over planes;
    // ga: 0 over H, 1 over W, contiguous rows of W over planes; gb: [H, W] contiguous, 0 over planes
    if (p.st[0][w] != 1 || p.st[0][h] != W) return false;
    if (p.st[1][h] != 0 || p.st[1][w] != 1) return false;
    if (p.st[2][h] != W || p.st[2][w] != 1) return false;
    if (p.st[3][h] != 0 || p.st[3][w] != 1) return false;
    if (p.st[4][h] != W || p.st[4][w] != 1) return false;
    int64_t P = 1, rowg = H * W, rowa = W;
    for (int d = h - 1; d >= 0; d--) {
        if (p.st[0][d] != rowg || p.st[2][d] != 0 || p.st[4][d] != 0 || p.st[3][d] != rowa) return false;
        rowg *= p.shape[d];
        rowa *= p.shape[d];
        P *= p.shape[d];
    }
    if (!aligned16(g) || !aligned16(b) || !aligned16(ga) || !aligned16(gb) || !aligned16(a)) return false;
    for (int d = 0; d < h; d++)
        if (p.st[1][d] % 4) return false;
    Prepared ap{};
    ap.nd = h;
    for (int d = 0; d < h; d++) {
        ap.shape[d] = p.shape[d];
        ap.st[0][d] = p.st[1][d];
    }
    make_map<1>(ap, 1, pl.amap);
    pl.P = (uint32_t)P;
    pl.H = (uint32_t)H;
    pl.W4 = (uint32_t)(W / 4);
    pl.T = (uint32_t)T;
    pl.nband = (uint32_t)nband;
    const int64_t blocks_per_cu = out == 2 || T >= 8 ? 1 : 2;
    const int64_t want = std::max<int64_t>(1, (int64_t)kPlanCUs * blocks_per_cu / nband);
    int64_t ranges = std::min<int64_t>(P, want);
    if (out & 1) {  // whole multiples of the resident workgroups until each range fits in res
        const int64_t fit = (int64_t)b2_res_groups(T) * (64 / (W / 4));
        const int64_t rounds = ((P + fit - 1) / fit + want - 1) / want;
        ranges = std::min<int64_t>(P, want * rounds);
    }
    // NC_HIP_BWD2_MAX_RANGES caps the plane ranges (more planes per workgroup): lets a small test
    // problem run the long-range paths (several wraps of the grad_a ring) that only large inputs reach
    if (const char *cap = getenv("NC_HIP_BWD2_MAX_RANGES"))
        if (atoll(cap) > 0) ranges = std::min<int64_t>(ranges, atoll(cap));
    pl.planes_per_block = (uint32_t)((P + ranges - 1) / ranges);
    pl.ranges = (uint32_t)((P + pl.planes_per_block - 1) / pl.planes_per_block);
    return true;
}

// workspace: grad_b partials [ranges][H*W] (when grad_b is written), then grad_a partials
// [P][nband][W] (when grad_a is written and a plane has several bands)
static size_t bwd2_gb_bytes(const Bwd2Plan &pl, int out) {
    return (out & 2) ? (size_t)pl.ranges * pl.H * pl.W4 * 4 * sizeof(double) : 0;
}
static size_t bwd2_ws(const Bwd2Plan &pl, int out = 3) {
    size_t n = bwd2_gb_bytes(pl, out);
    if ((out & 1) && pl.nband > 1) n += (size_t)pl.P * pl.nband * pl.W4 * 4 * sizeof(double);
    return n;
}

template <int MODE, int OUT>
static int launch_bwd2(const float *g, const float *a, const float *b, float *ga, float *gb, const Bwd2Plan &pl,
                       double alpha_b, int acc, int acc_b, void *ws, size_t ws_bytes, hipStream_t st) {
    const size_t need = bwd2_ws(pl, OUT);
    if (ws_bytes < need || (need && !ws))
        return set_error(NC_HIP_ERR_WORKSPACE, "binary_bwd2: workspace of %zu bytes needed, %zu given", need, ws_bytes);
    const uint32_t blocks = pl.ranges * pl.nband;
    double *gb_part = (OUT & 2) ? (double *)ws : nullptr;
    double *ga_part = ((OUT & 1) && pl.nband > 1) ? (double *)((char *)ws + bwd2_gb_bytes(pl, OUT)) : nullptr;
#define NC_B2_LAUNCH(TT)                                                                                          \
    if (acc)                                                                                                      \
        hipLaunchKernelGGL((k_bcast_bwd2<MODE, true, TT, OUT>), dim3(blocks), dim3(kB2), 0, st, g, a, b, ga,      \
                           ga_part, gb_part, pl, alpha_b);                                                        \
    else                                                                                                          \
        hipLaunchKernelGGL((k_bcast_bwd2<MODE, false, TT, OUT>), dim3(blocks), dim3(kB2), 0, st, g, a, b, ga,     \
                           ga_part, gb_part, pl, alpha_b)
    switch (pl.T) {
    case 1: NC_B2_LAUNCH(1); break;
    case 2: NC_B2_LAUNCH(2); break;
#if NC_B2_TMAX >= 4
    case 4: NC_B2_LAUNCH(4); break;
#endif
#if NC_B2_TMAX >= 8
    case 8: NC_B2_LAUNCH(8); break;
#endif
    default: return set_error(NC_HIP_ERR_ARG, "binary_bwd2: unsupported plan");
    }
#undef NC_B2_LAUNCH
    if ((OUT & 1) && pl.nband > 1) {
        const uint32_t n = pl.P * pl.W4 * 4;
        const unsigned grid = stream_grid(n, kB, 65536);  // one element per lane
        const IntDiv divW(pl.W4 * 4);
        if (acc) hipLaunchKernelGGL((k_bwd2_ga_combine<true>), dim3(grid), dim3(kB), 0, st, ga_part, ga, n, pl.W4 * 4, divW, pl.nband);
        else hipLaunchKernelGGL((k_bwd2_ga_combine<false>), dim3(grid), dim3(kB), 0, st, ga_part, ga, n, pl.W4 * 4, divW, pl.nband);
    }
    if (OUT & 2) {
        const uint32_t n = pl.H * pl.W4 * 4;
        if (acc_b) hipLaunchKernelGGL((k_bwd2_gb_combine<MODE, true>), dim3((n + 63) / 64), dim3(1024), 0, st, gb_part, b, gb, n, pl.ranges);
        else hipLaunchKernelGGL((k_bwd2_gb_combine<MODE, false>), dim3((n + 63) / 64), dim3(1024), 0, st, gb_part, b, gb, n, pl.ranges);
    }
    return check_launch("nc_hip_binary_bwd2");
}

// op -> kernel mode (add and sub share the kernel; sub scales grad_b by -1); acc applies to grad_a,
// acc_b to grad_b
template <int OUT>
static int launch_bwd2_op(int op, const float *g, const float *a, const float *b, float *ga, float *gb,
                          const Bwd2Plan &pl, int acc, int acc_b, void *ws, size_t ws_bytes, hipStream_t st) {
    const double alpha_b = op == NC_HIP_BIN_SUB ? -1.0 : 1.0;
    switch (op) {
    case NC_HIP_BIN_ADD:
    case NC_HIP_BIN_SUB: return launch_bwd2<0, OUT>(g, a, b, ga, gb, pl, alpha_b, acc, acc_b, ws, ws_bytes, st);
    case NC_HIP_BIN_MUL: return launch_bwd2<1, OUT>(g, a, b, ga, gb, pl, alpha_b, acc, acc_b, ws, ws_bytes, st);
    default: return launch_bwd2<3, OUT>(g, a, b, ga, gb, pl, alpha_b, acc, acc_b, ws, ws_bytes, st);
    }
}

// Layout of a contiguous gradient for an operand with broadcast strides sx over `shape`: stride 0
// where the operand is broadcast, row-major over its own dims elsewhere.
static void grad_layout(int nd, const int64_t *shape, const int64_t *sx, int64_t *out) {
    int64_t run = 1;
    for (int d = nd - 1; d >= 0; d--) {
        if (sx[d] == 0 && shape[d] != 1) {
            out[d] = 0;
        } else {
            out[d] = run;
            run *= shape[d];
        }
    }
}

// Workspace bound of the fused path for one gradient whose layout is sgx: the plan built as if the
// output were g[P, H, W] with H, W the last two dims (both operand layouts derived from sgx).
static size_t bwd2_single_ws_bound(int nd, const int64_t *shape, const int64_t *sgx) {
    if (nd < 3 || nd > NC_HIP_MAX_DIMS) return 0;
    int64_t cs[NC_HIP_MAX_DIMS], s = 1;
    for (int d = nd - 1; d >= 0; d--) {
        cs[d] = s;
        s *= shape[d];
    }
    // the two broadcast patterns of the fused kernel: a over [P, W] (0 over H), b over [H, W]
    int64_t sa[NC_HIP_MAX_DIMS], sb[NC_HIP_MAX_DIMS], run = 1;
    for (int d = nd - 1; d >= 0; d--) {
        const bool is_h = d == nd - 2;
        sa[d] = is_h ? 0 : run;
        if (!is_h) run *= shape[d];
    }
    run = 1;
    for (int d = nd - 1; d >= 0; d--) {
        const bool plane = d < nd - 2;
        sb[d] = plane ? 0 : run;
        if (!plane) run *= shape[d];
    }
    (void)sgx;
    const int64_t *strides[5] = {cs, sa, sb, sa, sb};
    Prepared p;
    if (prepare(nd, shape, 5, strides, p, "nc_hip_binary_bwd_workspace")) return 0;
    Bwd2Plan pl;
    const float *al = (const float *)(uintptr_t)256;
    return plan_bwd2(p, al, al, al, al, al, pl, 3) ? bwd2_ws(pl, 3) : 0;
}

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API int nc_hip_binary_fwd(int op, int nd, const int64_t *shape, const float *a,
                                            const int64_t *sa, const float *b, const int64_t *sb, float *o,
                                            const int64_t *so, void *stream) {
    Prepared p;
    const int64_t *strides[3] = {sa, sb, so};
    int rc = prepare(nd, shape, 3, strides, p, "nc_hip_binary_fwd");
    if (rc) return rc;
    if (p.numel && (!a || !b || !o)) return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_fwd: NULL pointer");
    hipStream_t st = as_stream(stream);
    switch (op) {
    case NC_HIP_BIN_ADD: return launch_fwd<NC_HIP_BIN_ADD>(a, b, o, p, st);
    case NC_HIP_BIN_SUB: return launch_fwd<NC_HIP_BIN_SUB>(a, b, o, p, st);
    case NC_HIP_BIN_MUL: return launch_fwd<NC_HIP_BIN_MUL>(a, b, o, p, st);
    case NC_HIP_BIN_DIV: return launch_fwd<NC_HIP_BIN_DIV>(a, b, o, p, st);
    default: return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_fwd: unknown op %d", op);
    }
}

static size_t bwd_workspace_run(int nd, const int64_t *shape, const int64_t *sgx);

// Broadcast gradients of 2^32 elements or more run as runs of at most 2^30 elements (for_each_run), so
// the workspace is the largest any run needs.
extern "C" NC_HIP_API size_t nc_hip_binary_bwd_workspace(int nd, const int64_t *shape, const int64_t *sgx) {
    if (nd < 0 || nd > NC_HIP_MAX_DIMS || !shape || !sgx) return 0;
    for (int d = 0; d < nd; d++)
        if (shape[d] < 0) return 0;
    const RunSplit rsp = run_split();
    if (numel_of(nd, shape) <= rsp.above) return bwd_workspace_run(nd, shape, sgx);
    size_t need = 0;
    const int64_t *st[1] = {sgx};
    for_each_run(nd, shape, 1, st, rsp.limit, [&](const int64_t *rs, const int64_t *, const bool *) {
        need = std::max(need, bwd_workspace_run(nd, rs, sgx));
        return 0;
    });
    return need;
}

static size_t bwd_workspace_run(int nd, const int64_t *shape, const int64_t *sgx) {
    // the plan depends only on the shape and on which dims gx keeps: use unit strides elsewhere
    int64_t cs[NC_HIP_MAX_DIMS], s = 1;
    for (int d = nd - 1; d >= 0; d--) {
        cs[d] = s;
        s *= shape[d];
    }
    const int64_t *strides[4] = {cs, cs, cs, sgx};
    Prepared p;
    if (prepare(nd, shape, 4, strides, p, "nc_hip_binary_bwd_workspace") || p.numel == 0) return 0;
    RedPlan pl;
    size_t need = 0;
    if (!plan_reduce(p, pl, &need)) need = 0;
    bool reduces = false;
    for (int d = 0; d < nd; d++) reduces |= sgx[d] == 0 && shape[d] != 1;
    // room for the fused single-pass kernel when the broadcast has its pattern
    if (reduces) need = std::max(need, bwd2_single_ws_bound(nd, shape, sgx));
    return need;
}

static int prepare_bwd2(int nd, const int64_t *shape, const int64_t *sg, const int64_t *sa, const int64_t *sb,
                        const int64_t *sga, const int64_t *sgb, Prepared &p);

// One operand's gradient through the fused kernel (the other output switched off), when the
// broadcast has its pattern and the workspace covers it.  Returns -1 when it does not apply.
static int try_bwd_fused_single(int op, int which, int nd, const int64_t *shape, const float *g, const int64_t *sg,
                                const float *a, const int64_t *sa, const float *b, const int64_t *sb, float *gx,
                                const int64_t *sgx, int accumulate, void *ws, size_t ws_bytes, hipStream_t st) {
    if (nd < 3 || nd > NC_HIP_MAX_DIMS) return -1;
    int64_t sgo[NC_HIP_MAX_DIMS];  // layout of the other (unwritten) gradient
    grad_layout(nd, shape, which == 0 ? sb : sa, sgo);
    const int64_t *sga = which == 0 ? sgx : sgo, *sgb = which == 0 ? sgo : sgx;
    const bool reads_ab = op == NC_HIP_BIN_MUL || op == NC_HIP_BIN_DIV;
    Prepared p;
    if (prepare_bwd2(nd, shape, sg, reads_ab ? sa : sga, reads_ab ? sb : sgb, sga, sgb, p) != NC_HIP_OK) return -1;
    Bwd2Plan pl;
    if (p.numel == 0 || !plan_bwd2(p, g, reads_ab ? a : gx, reads_ab ? b : gx, gx, gx, pl, which == 0 ? 1 : 2))
        return -1;
    const size_t need = bwd2_ws(pl, which == 0 ? 1 : 2);
    if (ws_bytes < need || (need && !ws)) return -1;
    if (which == 0) return launch_bwd2_op<1>(op, g, a, b, gx, nullptr, pl, accumulate, accumulate, ws, ws_bytes, st);
    if (reads_ab && NC_BIN_WARM) warm_operand(a, p, 1, st);  // grad_b's terms read a
    return launch_bwd2_op<2>(op, g, a, b, nullptr, gx, pl, accumulate, accumulate, ws, ws_bytes, st);
}

static int binary_bwd_run(int op, int which, int nd, const int64_t *shape, const float *g, const int64_t *sg,
                          const float *a, const int64_t *sa, const float *b, const int64_t *sb, float *gx,
                          const int64_t *sgx, int accumulate, void *ws, size_t ws_bytes, void *stream);

// Gradients of 2^32 elements or more: runs of at most 2^30 elements of g in index order, each through
// the ordinary paths; a run adds into what an earlier run wrote where gx is reduced over a cut dim.
extern "C" NC_HIP_API int nc_hip_binary_bwd(int op, int which, int nd, const int64_t *shape, const float *g,
                                            const int64_t *sg, const float *a, const int64_t *sa, const float *b,
                                            const int64_t *sb, float *gx, const int64_t *sgx, int accumulate,
                                            void *ws, size_t ws_bytes, void *stream) {
    if (op < 0 || op > 3 || (which != 0 && which != 1))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_bwd: bad op/which");
    if (nd < 0 || nd > NC_HIP_MAX_DIMS || !shape || !sg || !sa || !sb || !sgx)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_bwd: bad shape or strides");
    for (int d = 0; d < nd; d++)
        if (shape[d] < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_bwd: negative dim");
    const RunSplit rsp = run_split();
    if (numel_of(nd, shape) <= rsp.above)
        return binary_bwd_run(op, which, nd, shape, g, sg, a, sa, b, sb, gx, sgx, accumulate, ws, ws_bytes, stream);
    const int64_t *st[4] = {sg, sa, sb, sgx};
    return for_each_run(nd, shape, 4, st, rsp.limit, [&](const int64_t *rs, const int64_t *off, const bool *first) {
        return binary_bwd_run(op, which, nd, rs, adv(g, off[0]), sg, adv(a, off[1]), sa, adv(b, off[2]), sb,
                              adv(gx, off[3]), sgx, first[3] ? accumulate : 1, ws, ws_bytes, stream);
    });
}

static int binary_bwd_run(int op, int which, int nd, const int64_t *shape, const float *g, const int64_t *sg,
                          const float *a, const int64_t *sa, const float *b, const int64_t *sb, float *gx,
                          const int64_t *sgx, int accumulate, void *ws, size_t ws_bytes, void *stream) {
    Prepared p;
    int mode;
    float alpha;
    bool p1_is_a;
    int rc = prepare_grad(op, which, nd, shape, sg, sa, sb, sgx, p, mode, alpha, p1_is_a);
    if (rc) return rc;
    const float *p1 = p1_is_a ? a : b;
    const float *p2 = b;
    hipStream_t st = as_stream(stream);
    if (p.numel > 0) {
        rc = try_bwd_fused_single(op, which, nd, shape, g, sg, a, sa, b, sb, gx, sgx, accumulate, ws, ws_bytes, st);
        if (rc >= 0) return rc;
    }
    switch (mode) {
    case 0: return launch_grad<0>(g, g, g, gx, p, alpha, accumulate, ws, ws_bytes, st);
    case 1: return launch_grad<1>(g, p1, g, gx, p, alpha, accumulate, ws, ws_bytes, st);
    case 2: return launch_grad<2>(g, p1, g, gx, p, alpha, accumulate, ws, ws_bytes, st);
    default: return launch_grad<3>(g, p1, p2, gx, p, alpha, accumulate, ws, ws_bytes, st);
    }
}

static int prepare_bwd2(int nd, const int64_t *shape, const int64_t *sg, const int64_t *sa, const int64_t *sb,
                        const int64_t *sga, const int64_t *sgb, Prepared &p) {
    const int64_t *strides[5] = {sg, sa, sb, sga, sgb};
    return prepare(nd, shape, 5, strides, p, "nc_hip_binary_bwd2");
}

static size_t bwd2_workspace_run(int nd, const int64_t *shape, const int64_t *sga, const int64_t *sgb);

extern "C" NC_HIP_API size_t nc_hip_binary_bwd2_workspace(int nd, const int64_t *shape, const int64_t *sga,
                                                          const int64_t *sgb) {
    if (nd < 0 || nd > NC_HIP_MAX_DIMS || !shape) return 0;
    for (int d = 0; d < nd; d++)
        if (shape[d] < 0) return 0;
    const RunSplit rsp = run_split();
    if (numel_of(nd, shape) <= rsp.above) return bwd2_workspace_run(nd, shape, sga, sgb);
    size_t need = 0;
    const int64_t zeros[NC_HIP_MAX_DIMS] = {0, 0, 0, 0, 0, 0};
    const int64_t *st[1] = {zeros};
    for_each_run(nd, shape, 1, st, rsp.limit, [&](const int64_t *rs, const int64_t *, const bool *) {
        need = std::max(need, bwd2_workspace_run(nd, rs, sga, sgb));
        return 0;
    });
    return need;
}

static size_t bwd2_workspace_run(int nd, const int64_t *shape, const int64_t *sga, const int64_t *sgb) {
    size_t wa = sga ? nc_hip_binary_bwd_workspace(nd, shape, sga) : 0;
    size_t wb = sgb ? nc_hip_binary_bwd_workspace(nd, shape, sgb) : 0;
    size_t need = wa > wb ? wa : wb;
    if (sga && sgb && nd >= 2 && nd <= NC_HIP_MAX_DIMS) {
        // the fused plan depends on shape and grad layouts; model g, b as contiguous, a as broadcast like ga
        int64_t cs[NC_HIP_MAX_DIMS], s = 1;
        for (int d = nd - 1; d >= 0; d--) {
            cs[d] = s;
            s *= shape[d];
        }
        Prepared p;
        if (prepare_bwd2(nd, shape, cs, sga, sgb, sga, sgb, p) == NC_HIP_OK) {
            Bwd2Plan pl;
            const float *al = (const float *)(uintptr_t)256;  // any 16-byte aligned address: only the plan is needed
            if (plan_bwd2(p, al, al, al, al, al, pl, 3)) need = std::max(need, bwd2_ws(pl));
        }
    }
    return need;
}

static int binary_bwd2_run(int op, int nd, const int64_t *shape, const float *g, const int64_t *sg,
                           const float *a, const int64_t *sa, const float *b, const int64_t *sb, float *ga,
                           const int64_t *sga, float *gb, const int64_t *sgb, int acc_a, int acc_b, void *ws,
                           size_t ws_bytes, void *stream);

// Both gradients of 2^32 elements or more: runs of at most 2^30 elements of g in index order (each the
// one-pass kernel where the broadcast has its pattern); grad_a and grad_b each add into what an earlier
// run wrote where they are reduced over a cut dim (config-sized a[256,512,1,64] + b[1,1,512,64]: four
// runs of 64 planes; grad_a written by each, grad_b stored by the first and added to by the rest).
extern "C" NC_HIP_API int nc_hip_binary_bwd2(int op, int nd, const int64_t *shape, const float *g,
                                             const int64_t *sg, const float *a, const int64_t *sa, const float *b,
                                             const int64_t *sb, float *ga, const int64_t *sga, float *gb,
                                             const int64_t *sgb, int accumulate, void *ws, size_t ws_bytes,
                                             void *stream) {
    if (op < 0 || op > 3) return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_bwd2: bad op");
    if (nd < 0 || nd > NC_HIP_MAX_DIMS || !shape || !sg || !sa || !sb || (ga && !sga) || (gb && !sgb))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_bwd2: bad shape or strides");
    for (int d = 0; d < nd; d++)
        if (shape[d] < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_binary_bwd2: negative dim");
    const RunSplit rsp = run_split();
    if (numel_of(nd, shape) <= rsp.above)
        return binary_bwd2_run(op, nd, shape, g, sg, a, sa, b, sb, ga, sga, gb, sgb, accumulate, accumulate, ws,
                               ws_bytes, stream);
    const int64_t zeros[NC_HIP_MAX_DIMS] = {0, 0, 0, 0, 0, 0};
    const int64_t *st[5] = {sg, sa, sb, ga ? sga : zeros, gb ? sgb : zeros};
    return for_each_run(nd, shape, 5, st, rsp.limit, [&](const int64_t *rs, const int64_t *off, const bool *first) {
        return binary_bwd2_run(op, nd, rs, adv(g, off[0]), sg, adv(a, off[1]), sa, adv(b, off[2]), sb,
                               adv(ga, off[3]), sga, adv(gb, off[4]), sgb, first[3] ? accumulate : 1,
                               first[4] ? accumulate : 1, ws, ws_bytes, stream);
    });
}

static int binary_bwd2_run(int op, int nd, const int64_t *shape, const float *g, const int64_t *sg,
                           const float *a, const int64_t *sa, const float *b, const int64_t *sb, float *ga,
                           const int64_t *sga, float *gb, const int64_t *sgb, int acc_a, int acc_b, void *ws,
                           size_t ws_bytes, void *stream) {
    if (ga && gb) {
        // add / sub read neither operand: plan with the gradients' layouts in their place
        const bool reads_ab = op == NC_HIP_BIN_MUL || op == NC_HIP_BIN_DIV;
        Prepared p;
        int rc = prepare_bwd2(nd, shape, sg, reads_ab ? sa : sga, reads_ab ? sb : sgb, sga, sgb, p);
        if (rc) return rc;
        Bwd2Plan pl;
        if (p.numel > 0 && plan_bwd2(p, g, reads_ab ? a : ga, reads_ab ? b : gb, ga, gb, pl, 3)) {
            if (reads_ab && NC_BIN_WARM) warm_operand(a, p, 1, as_stream(stream));  // grad_b's terms read a
            return launch_bwd2_op<3>(op, g, a, b, ga, gb, pl, acc_a, acc_b, ws, ws_bytes, as_stream(stream));
        }
    }
    int rc = NC_HIP_OK;
    if (ga) rc = binary_bwd_run(op, 0, nd, shape, g, sg, a, sa, b, sb, ga, sga, acc_a, ws, ws_bytes, stream);
    if (rc == NC_HIP_OK && gb)
        rc = binary_bwd_run(op, 1, nd, shape, g, sg, a, sa, b, sb, gb, sgb, acc_b, ws, ws_bytes, stream);
    return rc;
}

// ------------------------------------------------------------------------------------------------
// strided copies, fills, conversions
// ------------------------------------------------------------------------------------------------
namespace nchip {

template <typename T>
__global__ __launch_bounds__(kB) void k_gather(const T *__restrict__ src, T *__restrict__ dst, IdxMap<1> m,
                                               uint32_t n) {
    const uint32_t step = gridDim.x * kB;
    for (uint32_t w = blockIdx.x * kB + threadIdx.x; w < n; w += step) {
        int64_t off[1];
        offsets<1>(m, w, off);
        dst[w] = src[off[0]];
    }
}

__global__ __launch_bounds__(kB) void k_scatter_add(const float *__restrict__ src, float *__restrict__ dst,
                                                    IdxMap<1> m, uint32_t n) {
    const uint32_t step = gridDim.x * kB;
    for (uint32_t w = blockIdx.x * kB + threadIdx.x; w < n; w += step) {
        int64_t off[1];
        offsets<1>(m, w, off);
        dst[off[0]] = dst[off[0]] + src[w];
    }
}

__global__ __launch_bounds__(kB) void k_axpy(const float *__restrict__ x, float *__restrict__ y, int64_t n, float al) {
    const int64_t step = (int64_t)gridDim.x * kB;
    for (int64_t i = (int64_t)blockIdx.x * kB + threadIdx.x; i < n; i += step) y[i] = fma_(al, x[i], y[i]);
}

template <typename T>
__global__ __launch_bounds__(kB) void k_fill(T *__restrict__ dst, T v, int64_t n) {
    const int64_t step = (int64_t)gridDim.x * kB;
    for (int64_t i = (int64_t)blockIdx.x * kB + threadIdx.x; i < n; i += step) dst[i] = v;
}

// 16-byte pattern fill: one non-temporal 128-bit store per lane, 64-lane workgroups over the whole
// range (the streaming shape that reaches the write ceiling)
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(64) void k_fill16(u4v *__restrict__ dst, u4v v, int64_t n16) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (i < n16) __builtin_nontemporal_store(v, dst + i);
}

__global__ void k_add_at(float *p, float v) { p[0] = p[0] + v; }

template <typename S>
__device__ __forceinline__ double load_d(const S *p, int64_t i) { return (double)p[i]; }

__device__ __forceinline__ double saturate(double v, double lo, double hi) {
    if (v != v) return 0.0;
    return v < lo ? lo : v > hi ? hi : v;
}

template <typename S, typename D>
__global__ __launch_bounds__(kB) void k_convert(const S *__restrict__ src, D *__restrict__ dst, int64_t n) {
    const int64_t step = (int64_t)gridDim.x * kB;
    for (int64_t i = (int64_t)blockIdx.x * kB + threadIdx.x; i < n; i += step) {
        const double v = (double)src[i];
        if constexpr (sizeof(D) == 4 && D(0.5) != D(0)) dst[i] = (float)v;                 // f32
        else if constexpr (sizeof(D) == 4) dst[i] = (int32_t)saturate(v, -2147483648.0, 2147483647.0);
        else if constexpr (D(-1) < D(0)) dst[i] = (int8_t)saturate(v, -128.0, 127.0);       // i8
        else dst[i] = (uint8_t)saturate(v, 0.0, 255.0);                                     // u8
    }
}

}  // namespace nchip

// row-major (contiguous) element strides of shape
static void contiguous_strides(int nd, const int64_t *shape, int64_t *cs) {
    int64_t s = 1;
    for (int d = nd - 1; d >= 0; d--) {
        cs[d] = s;
        s *= shape[d];
    }
}

// Gathers of 2^32 elements or more: runs of at most 2^30 elements (for_each_run), each a launch of
// its own; the destination is the contiguous tensor of the whole shape.
extern "C" NC_HIP_API int nc_hip_copy_strided(int elem_bytes, int nd, const int64_t *shape, const void *src,
                                              const int64_t *ss, void *dst, void *stream) {
    Prepared p;
    const int64_t *strides[1] = {ss};
    int rc = prepare(nd, shape, 1, strides, p, "nc_hip_copy_strided");
    if (rc) return rc;
    if (p.numel == 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    if (p.nd <= 1 && (p.nd == 0 || p.st[0][0] == 1)) {
        if (hipMemcpyAsync(dst, src, (size_t)p.numel * elem_bytes, hipMemcpyDeviceToDevice, st) != hipSuccess)
            return check_launch("nc_hip_copy_strided");
        return NC_HIP_OK;
    }
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
        return set_error(NC_HIP_ERR_ARG, "copy_strided: element size %d", elem_bytes);
    const RunSplit rsp = run_split();
    if (p.numel > rsp.above) {
        int64_t cs[NC_HIP_MAX_DIMS];
        contiguous_strides(nd, shape, cs);
        const int64_t *st2[2] = {ss, cs};
        return for_each_run(nd, shape, 2, st2, rsp.limit, [&](const int64_t *rs, const int64_t *off, const bool *) {
            return nc_hip_copy_strided(elem_bytes, nd, rs, (const char *)src + off[0] * elem_bytes, ss,
                                       (char *)dst + off[1] * elem_bytes, stream);
        });
    }
    IdxMap<1> m;
    make_map<1>(p, 1, m);
    const unsigned grid = stream_grid(p.numel, kB, 16);
    const uint32_t n = (uint32_t)p.numel;
    switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(k_gather<uint8_t>, grid, kB, 0, st, (const uint8_t *)src, (uint8_t *)dst, m, n); break;
    case 2: hipLaunchKernelGGL(k_gather<uint16_t>, grid, kB, 0, st, (const uint16_t *)src, (uint16_t *)dst, m, n); break;
    case 4: hipLaunchKernelGGL(k_gather<uint32_t>, grid, kB, 0, st, (const uint32_t *)src, (uint32_t *)dst, m, n); break;
    case 8: hipLaunchKernelGGL(k_gather<uint64_t>, grid, kB, 0, st, (const uint64_t *)src, (uint64_t *)dst, m, n); break;
    default: return set_error(NC_HIP_ERR_ARG, "copy_strided: element size %d", elem_bytes);
    }
    return check_launch("nc_hip_copy_strided");
}

extern "C" NC_HIP_API int nc_hip_accumulate_strided(int nd, const int64_t *shape, const float *src, float *dst,
                                                    const int64_t *sd, void *stream) {
    Prepared p;
    const int64_t *strides[1] = {sd};
    int rc = prepare(nd, shape, 1, strides, p, "nc_hip_accumulate_strided");
    if (rc) return rc;
    if (p.numel == 0) return NC_HIP_OK;
    const RunSplit rsp = run_split();
    if (p.numel > rsp.above) {  // runs of at most 2^30 elements; src is contiguous over shape
        int64_t cs[NC_HIP_MAX_DIMS];
        contiguous_strides(nd, shape, cs);
        const int64_t *st2[2] = {cs, sd};
        return for_each_run(nd, shape, 2, st2, rsp.limit, [&](const int64_t *rs, const int64_t *off, const bool *) {
            return nc_hip_accumulate_strided(nd, rs, src + off[0], dst + off[1], sd, stream);
        });
    }
    if (p.nd == 0) {
        p.nd = 1;
        p.shape[0] = 1;
        p.st[0][0] = 0;
    }
    IdxMap<1> m;
    make_map<1>(p, 1, m);
    hipLaunchKernelGGL(k_scatter_add, stream_grid(p.numel, kB, 16), kB, 0, as_stream(stream), src, dst, m,
                       (uint32_t)p.numel);
    return check_launch("nc_hip_accumulate_strided");
}

extern "C" NC_HIP_API int nc_hip_axpy(int64_t n, float alpha, const float *x, float *y, void *stream) {
    if (n <= 0) return NC_HIP_OK;
    hipLaunchKernelGGL(k_axpy, stream_grid(n, kB, 16), kB, 0, as_stream(stream), x, y, n, alpha);
    return check_launch("nc_hip_axpy");
}

extern "C" NC_HIP_API int nc_hip_fill(void *dst, int elem_bytes, uint64_t pattern, int64_t n, void *stream) {
    if (n <= 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    if ((elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8) && aligned16(dst) &&
        n * elem_bytes >= 16) {
        // whole 16-byte blocks with the pattern repeated, then the tail elements below
        uint64_t w = pattern;
        if (elem_bytes == 1) w = (w & 0xffu) * 0x0101010101010101ull;
        else if (elem_bytes == 2) w = (w & 0xffffu) * 0x0001000100010001ull;
        else if (elem_bytes == 4) w = (w & 0xffffffffu) * 0x0000000100000001ull;
        const u4v v{(uint32_t)w, (uint32_t)(w >> 32), (uint32_t)w, (uint32_t)(w >> 32)};
        const int64_t n16 = n * elem_bytes / 16;
        const int64_t blocks = (n16 + 63) / 64;
        for (int64_t b0 = 0; b0 < blocks; b0 += INT32_MAX / 2) {  // launches of < 2^30 workgroups
            const int64_t nb = std::min<int64_t>(blocks - b0, INT32_MAX / 2);
            hipLaunchKernelGGL(k_fill16, dim3((unsigned)nb), dim3(64), 0, st, (u4v *)dst + b0 * 64,
                               v, std::min<int64_t>(n16 - b0 * 64, nb * 64));
        }
        const int64_t done = n16 * 16 / elem_bytes;
        if (done == n) return check_launch("nc_hip_fill");
        dst = (char *)dst + done * elem_bytes;
        n -= done;
    }
    const unsigned grid = stream_grid(n, kB, 16);
    switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(k_fill<uint8_t>, grid, kB, 0, st, (uint8_t *)dst, (uint8_t)pattern, n); break;
    case 2: hipLaunchKernelGGL(k_fill<uint16_t>, grid, kB, 0, st, (uint16_t *)dst, (uint16_t)pattern, n); break;
    case 4: hipLaunchKernelGGL(k_fill<uint32_t>, grid, kB, 0, st, (uint32_t *)dst, (uint32_t)pattern, n); break;
    case 8: hipLaunchKernelGGL(k_fill<uint64_t>, grid, kB, 0, st, (uint64_t *)dst, (uint64_t)pattern, n); break;
    default: return set_error(NC_HIP_ERR_ARG, "fill: element size %d", elem_bytes);
    }
    return check_launch("nc_hip_fill");
}

extern "C" NC_HIP_API int nc_hip_add_scalar_at(float *p, float v, void *stream) {
    hipLaunchKernelGGL(k_add_at, 1, 1, 0, as_stream(stream), p, v);
    return check_launch("nc_hip_add_scalar_at");
}

extern "C" NC_HIP_API int nc_hip_convert(int from, int to, int64_t n, const void *src, void *dst, void *stream) {
    if (n <= 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    const unsigned grid = stream_grid(n, kB, 16);
#define NC_CONV(S, D) hipLaunchKernelGGL((k_convert<S, D>), grid, kB, 0, st, (const S *)src, (D *)dst, n)
#define NC_CONV_TO(S)                                          \
    switch (to) {                                              \
    case NC_HIP_F32: NC_CONV(S, float); break;                 \
    case NC_HIP_I32: NC_CONV(S, int32_t); break;               \
    case NC_HIP_I8: NC_CONV(S, int8_t); break;                 \
    case NC_HIP_U8: NC_CONV(S, uint8_t); break;                \
    default: return set_error(NC_HIP_ERR_ARG, "convert: target %d", to); \
    }
    switch (from) {
    case NC_HIP_F32: NC_CONV_TO(float); break;
    case NC_HIP_I32: NC_CONV_TO(int32_t); break;
    case NC_HIP_I8: NC_CONV_TO(int8_t); break;
    case NC_HIP_U8: NC_CONV_TO(uint8_t); break;
    default: return set_error(NC_HIP_ERR_ARG, "convert: source %d", from);
    }
#undef NC_CONV_TO
#undef NC_CONV
    return check_launch("nc_hip_convert");
}

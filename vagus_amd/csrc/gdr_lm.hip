// Two small kernels of the language model's one-token decode step around the
// layer kernels, each replacing a run of torch's elementwise kernels:
//
//  * scalar_gates_kernel: the scalar gate and the beta logits of one decode
//    token (GatedDeltaNet._gates, linear_attention.py:719-721 and :734-735):
//    the projections W_a x and W_b x (rounded to the element type, as the
//    module's nn.Linear returns them), then
//        g    = -exp(A_log) * softplus(W_a x + dt_bias)      (fp32)
//        beta = W_b x                                         (fp32, the logits)
//    -exp(A_log) comes in precomputed.  The projections are 2H dot products of
//    dim elements per token: a wavefront owns eight of them, its lanes split
//    the row, and a shuffle reduction closes each one.
//
//  * swiglu_kernel: the FFN's SiLU(x1) x xgate (infra/components/ffn.py:48-50)
//    over [rows, 2 h] -> [rows, h], with the module's two roundings: SiLU's
//    result in the element type, then the product.
//
// Both use the accurate expf / log1pf, as torch's softplus and SiLU do.
#include <type_traits>

#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

namespace {

// torch's softplus at beta 1, threshold 20
__device__ __forceinline__ float softplus_t(float x) { return x > 20.f ? x : log1pf(expf(x)); }

}  // namespace

// One wavefront per (token, OPW outputs): every lane loads its slice of the
// row and of the OPW weight rows at once, so the call costs about one trip to
// memory rather than one per output.
constexpr int GATE_OPW = 8;

template <typename E>
__global__ void __launch_bounds__(64) scalar_gates_kernel(const E *__restrict__ x, const E *__restrict__ w,
                                                          const float *__restrict__ neg_a,
                                                          const float *__restrict__ dt_bias, float *g, float *beta,
                                                          int dim, int H, int n_out) {
    constexpr int VE = 16 / (int)sizeof(E);
    typedef E V __attribute__((ext_vector_type(VE)));
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int n0 = blockIdx.y * GATE_OPW;
    const int nu = dim / VE;
    const E *xr = x + row * dim;
    float acc[GATE_OPW];
#pragma unroll
    for (int j = 0; j < GATE_OPW; ++j) acc[j] = 0.f;
#pragma unroll 2
    for (int u = lane; u < nu; u += 64) {
        const V xv = *reinterpret_cast<const V *>(xr + (int64_t)u * VE);
        V wv[GATE_OPW];
#pragma unroll
        for (int j = 0; j < GATE_OPW; ++j) {
            const int n = n0 + j < n_out ? n0 + j : n_out - 1;            // rows past the end: reread the last
            wv[j] = *reinterpret_cast<const V *>(w + (int64_t)n * dim + (int64_t)u * VE);
        }
#pragma unroll
        for (int j = 0; j < GATE_OPW; ++j)
#pragma unroll
            for (int e = 0; e < VE; ++e) acc[j] += (float)xv[e] * (float)wv[j][e];
    }
#pragma unroll
    for (int j = 0; j < GATE_OPW; ++j) {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) acc[j] += __shfl_xor(acc[j], m);
    }
    if (lane < GATE_OPW && n0 + lane < n_out) {
        float a = acc[0];
#pragma unroll
        for (int j = 1; j < GATE_OPW; ++j) a = lane == j ? acc[j] : a;
        const int n = n0 + lane;
        const float p = (float)(E)a;                                      // nn.Linear's output in E
        if (n < H) g[row * H + n] = neg_a[n] * softplus_t(p + dt_bias[n]);
        else beta[row * H + (n - H)] = p;
    }
}

template <typename E>
__global__ void __launch_bounds__(256) swiglu_kernel(const E *__restrict__ x, E *__restrict__ y, int64_t rows,
                                                     int hidden) {
    constexpr int VE = 16 / (int)sizeof(E);
    typedef E V __attribute__((ext_vector_type(VE)));
    const int nu = hidden / VE;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * nu) return;
    const int64_t row = i / nu;
    const int u = (int)(i - row * nu);
    const E *xr = x + row * 2 * (int64_t)hidden;
    const V a = *reinterpret_cast<const V *>(xr + (int64_t)u * VE);
    const V b = *reinterpret_cast<const V *>(xr + hidden + (int64_t)u * VE);
    V o;
#pragma unroll
    for (int e = 0; e < VE; ++e) {
        const float s = (float)a[e] / (1.f + expf(-(float)a[e]));
        o[e] = (E)((float)(E)s * (float)b[e]);
    }
    *reinterpret_cast<V *>(y + row * (int64_t)hidden + (int64_t)u * VE) = o;
}

template <typename E>
static hipError_t scalar_gates_t(const void *x, const void *w, const float *neg_a, const float *dt_bias, float *g,
                                 float *beta, int64_t rows, int dim, int H, bool with_beta, hipStream_t stream) {
    const int n_out = with_beta ? 2 * H : H;
    hipLaunchKernelGGL((scalar_gates_kernel<E>), dim3((unsigned)rows, (unsigned)((n_out + GATE_OPW - 1) / GATE_OPW)),
                       dim3(64), 0, stream,
                       reinterpret_cast<const E *>(x), reinterpret_cast<const E *>(w), neg_a, dt_bias, g, beta, dim,
                       H, n_out);
    return hipGetLastError();
}

hipError_t scalar_gates(int dtype, const void *x, const void *w, const float *neg_a, const float *dt_bias, float *g,
                        float *beta, int64_t rows, int dim, int H, bool with_beta, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (dtype == 1) return scalar_gates_t<__bf16>(x, w, neg_a, dt_bias, g, beta, rows, dim, H, with_beta, stream);
    if (dtype == 2) return scalar_gates_t<_Float16>(x, w, neg_a, dt_bias, g, beta, rows, dim, H, with_beta, stream);
    return scalar_gates_t<float>(x, w, neg_a, dt_bias, g, beta, rows, dim, H, with_beta, stream);
}

template <typename E>
static hipError_t swiglu_t(const void *x, void *y, int64_t rows, int hidden, hipStream_t stream) {
    constexpr int VE = 16 / (int)sizeof(E);
    const int64_t blocks = (rows * (hidden / VE) + 255) / 256;
    hipLaunchKernelGGL((swiglu_kernel<E>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<const E *>(x), reinterpret_cast<E *>(y), rows, hidden);
    return hipGetLastError();
}

hipError_t swiglu(int dtype, const void *x, void *y, int64_t rows, int hidden, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (dtype == 1) return swiglu_t<__bf16>(x, y, rows, hidden, stream);
    if (dtype == 2) return swiglu_t<_Float16>(x, y, rows, hidden, stream);
    return swiglu_t<float>(x, y, rows, hidden, stream);
}

}  // namespace vgdr

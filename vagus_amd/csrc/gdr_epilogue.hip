// The layer's output epilogue, RMSNorm(o) x SiLU(gate) over the value head
// dim (linear_attention.py:814-825, norm_layer.py:15-24), as one HBM pass.
//
// Rows of dv elements (one per (token, head)) are cut into 16-byte units; a
// group of LPR = dv / VE consecutive lanes owns one row, so a wavefront covers
// 64 / LPR rows and every global access is one coalesced 16-byte load or
// store.  The sum of squares is reduced across the group with xor shuffles.
// The decode step applies the same epilogue inside recurrent_kernel, where a
// workgroup holds a whole row; the chunk kernels tile dv across workgroups,
// so prefill runs this pass after the scan.
#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

__device__ __forceinline__ float silu_(float x) { return x * sigmoidf_(x); }

template <typename E, int LPR>
__global__ void __launch_bounds__(256) norm_gate_kernel(const E *o, const E *__restrict__ gate,
                                                        const void *__restrict__ gamma, int gamma_f32, float eps,
                                                        E *out, int64_t n_rows) {
    constexpr int VE = 16 / (int)sizeof(E), DV = LPR * VE;
    typedef E V __attribute__((ext_vector_type(VE)));
    const int64_t gt = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = gt / LPR;
    const int part = (int)(gt % LPR);
    const bool live = row < n_rows;
    const int64_t off = (live ? row : n_rows - 1) * DV + part * VE;      // groups past the end re-read the last row
    // o and the gate stream through once: nontemporal
    const V xv = __builtin_nontemporal_load(reinterpret_cast<const V *>(o + off));
    const V gv = __builtin_nontemporal_load(reinterpret_cast<const V *>(gate + off));
    float x[VE], w[VE];
    float ss = 0.f;
    if (gamma_f32) {
        // VE fp32 values: one or two 16-byte loads (gamma is 16-byte aligned)
        const f32x4 *gp = reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(gamma) + part * VE);
#pragma unroll
        for (int q = 0; q < VE / 4; ++q) {
            const f32x4 g4 = gp[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) w[4 * q + e] = g4[e];
        }
    } else {
        const V g = *reinterpret_cast<const V *>(reinterpret_cast<const E *>(gamma) + part * VE);
#pragma unroll
        for (int e = 0; e < VE; ++e) w[e] = (float)g[e];
    }
#pragma unroll
    for (int e = 0; e < VE; ++e) {
        x[e] = (float)xv[e];
        ss += x[e] * x[e];
    }
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) ss += __shfl_xor(ss, m);
    const float r = rsqrtf(ss * (1.f / DV) + eps);
    V y;
#pragma unroll
    for (int e = 0; e < VE; ++e) y[e] = (E)(x[e] * r * w[e] * silu_((float)gv[e]));
    if (live) __builtin_nontemporal_store(y, reinterpret_cast<V *>(out + off));
}

template <typename E>
static hipError_t norm_gate_t(const void *o, const Epilogue &ep, void *out, int64_t n_rows, int dv,
                              hipStream_t stream) {
    constexpr int VE = 16 / (int)sizeof(E);
    const int lpr = dv / VE;
    const int64_t blocks = (n_rows * lpr + 255) / 256;
    if (blocks == 0) return hipSuccess;
    const E *x = reinterpret_cast<const E *>(o), *g = reinterpret_cast<const E *>(ep.gate);
    E *y = reinterpret_cast<E *>(out);
#define VGDR_NG(L)                                                                                             \
    case L:                                                                                                     \
        hipLaunchKernelGGL((norm_gate_kernel<E, L>), dim3((unsigned)blocks), dim3(256), 0, stream, x, g, ep.gamma, \
                           ep.gamma_f32, ep.eps, y, n_rows);                                                    \
        break;
    switch (lpr) {
        VGDR_NG(1) VGDR_NG(2) VGDR_NG(4) VGDR_NG(8) VGDR_NG(16) VGDR_NG(32) VGDR_NG(64)
        default: return hipErrorInvalidValue;
    }
#undef VGDR_NG
    return hipGetLastError();
}

hipError_t norm_gate(int dtype, const void *o, const Epilogue &ep, void *out, int64_t n_rows, int dv,
                     hipStream_t stream) {
    if (dtype == 1) return norm_gate_t<__bf16>(o, ep, out, n_rows, dv, stream);
    if (dtype == 2) return norm_gate_t<_Float16>(o, ep, out, n_rows, dv, stream);
    return norm_gate_t<float>(o, ep, out, n_rows, dv, stream);
}

// The pre-norm blocks' RMSNorm (norm_layer.py:15-23) with the residual add in
// front of it (block.py:57-59, :85-87): h = x + res rounded to E (the stream's
// new value, stored to x_out), then y = E(E(h * rsqrt(mean(h^2) + eps)) * gamma),
// the module's order of roundings.  One workgroup per row; a thread holds up to U
// 16-byte units of the row in registers between the two passes.  Decode feeds
// a handful of rows of a few thousand elements, so one kernel here replaces the
// eight elementwise and reduction kernels of the module's expression.
template <typename E, int U>
// x_out may be x or res itself (the residual stream updated in place), so
// neither input is declared __restrict__.
__global__ void __launch_bounds__(256) rms_norm_kernel(const E *x, const E *res, E *x_out,
                                                       const E *__restrict__ gamma, float eps, E *y, int dim) {
    constexpr int VE = 16 / (int)sizeof(E);
    typedef E V __attribute__((ext_vector_type(VE)));
    __shared__ float part[4];
    const int tid = threadIdx.x, nu = dim / VE;
    const int64_t base = (int64_t)blockIdx.x * dim;
    float h[U][VE];
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = tid + 256 * u;
        if (i < nu) {
            V hv = *reinterpret_cast<const V *>(x + base + (int64_t)i * VE);
            if (res) {
                const V rv = *reinterpret_cast<const V *>(res + base + (int64_t)i * VE);
#pragma unroll
                for (int e = 0; e < VE; ++e) hv[e] = (E)((float)hv[e] + (float)rv[e]);
            }
            if (x_out) *reinterpret_cast<V *>(x_out + base + (int64_t)i * VE) = hv;
#pragma unroll
            for (int e = 0; e < VE; ++e) {
                h[u][e] = (float)hv[e];
                ss += h[u][e] * h[u][e];
            }
        }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) ss += __shfl_xor(ss, m);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float r = rsqrtf((part[0] + part[1] + part[2] + part[3]) / (float)dim + eps);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = tid + 256 * u;
        if (i < nu) {
            const V gv = *reinterpret_cast<const V *>(gamma + (int64_t)i * VE);
            V o;
#pragma unroll
            for (int e = 0; e < VE; ++e) o[e] = (E)((float)(E)(h[u][e] * r) * (float)gv[e]);
            *reinterpret_cast<V *>(y + base + (int64_t)i * VE) = o;
        }
    }
}

template <typename E>
static hipError_t rms_norm_t(const void *x, const void *res, void *x_out, const void *gamma, void *y, int64_t rows,
                             int dim, float eps, hipStream_t stream) {
    constexpr int VE = 16 / (int)sizeof(E);
    const int units = dim / VE;
    const E *xe = reinterpret_cast<const E *>(x), *re = reinterpret_cast<const E *>(res),
            *ge = reinterpret_cast<const E *>(gamma);
    E *xo = reinterpret_cast<E *>(x_out), *ye = reinterpret_cast<E *>(y);
    const dim3 grid((unsigned)rows);
    if (units <= 256)
        hipLaunchKernelGGL((rms_norm_kernel<E, 1>), grid, dim3(256), 0, stream, xe, re, xo, ge, eps, ye, dim);
    else if (units <= 512)
        hipLaunchKernelGGL((rms_norm_kernel<E, 2>), grid, dim3(256), 0, stream, xe, re, xo, ge, eps, ye, dim);
    else if (units <= 1024)
        hipLaunchKernelGGL((rms_norm_kernel<E, 4>), grid, dim3(256), 0, stream, xe, re, xo, ge, eps, ye, dim);
    else
        hipLaunchKernelGGL((rms_norm_kernel<E, 8>), grid, dim3(256), 0, stream, xe, re, xo, ge, eps, ye, dim);
    return hipGetLastError();
}

hipError_t rms_norm(int dtype, const void *x, const void *res, void *x_out, const void *gamma, void *y, int64_t rows,
                    int dim, float eps, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (dtype == 1) return rms_norm_t<__bf16>(x, res, x_out, gamma, y, rows, dim, eps, stream);
    if (dtype == 2) return rms_norm_t<_Float16>(x, res, x_out, gamma, y, rows, dim, eps, stream);
    return rms_norm_t<float>(x, res, x_out, gamma, y, rows, dim, eps, stream);
}

}  // namespace vgdr

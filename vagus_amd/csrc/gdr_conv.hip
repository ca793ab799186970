// The layer's short causal convolution + SiLU over a whole call's tokens
// (ShortConv, opt.py:15-100; fla's causal_conv1d as the reference calls it,
// :73-77), for prefill.  The decode kernel applies the same convolution per
// token; here it is one HBM pass over x.
//
// A thread owns VE = 16 / sizeof(E) consecutive channels (one 16-byte unit)
// for a run of RUN consecutive tokens, so a wavefront reads 64 neighbouring
// units of one token row per load.  The K - 1 inputs before the current token
// stay in registers as a sliding window: each input unit is loaded once per
// run (plus K - 1 at the run's start).  Inputs before a sequence's first token
// come from its conv cache [K, D] (the previous call's last K inputs,
// linear_attention.py:929-941) or are zero; a run that crosses into the next
// packed segment restarts its window there.
#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

namespace {

constexpr int RUN = 16;

template <typename E>
struct Unit {
    static constexpr int VE = 16 / (int)sizeof(E);
    typedef E V __attribute__((ext_vector_type(VE)));
    float f[VE];
    __device__ __forceinline__ void load(const E *p) {
        const V v = *reinterpret_cast<const V *>(p);
#pragma unroll
        for (int e = 0; e < VE; ++e) f[e] = (float)v[e];
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int e = 0; e < VE; ++e) f[e] = 0.f;
    }
};

__device__ __forceinline__ int64_t clamp_tok(int32_t c, int64_t n_tokens) {
    return c < 0 ? 0 : (c > n_tokens ? n_tokens : c);
}

// the segment holding token t: the last s with cu[s] <= t (segments clamped into [0, n_tokens])
__device__ __forceinline__ int seg_at(const int32_t *cu, int n, int64_t n_tokens, int64_t t) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (clamp_tok(cu[mid], n_tokens) <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

}  // namespace

template <typename E, int K>
__global__ void __launch_bounds__(256) causal_conv_kernel(const ConvParams p) {
    using U = Unit<E>;
    constexpr int VE = U::VE;
    const int64_t ncg = p.D / VE;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t cg = gid % ncg, run = gid / ncg;
    const int64_t t0 = run * RUN;
    if (t0 >= p.n_tokens) return;
    const int64_t c0 = cg * VE;
    const E *x = reinterpret_cast<const E *>(p.x);
    const E *st = reinterpret_cast<const E *>(p.state_in);
    E *y = reinterpret_cast<E *>(p.y);

    float w[K][VE];
#pragma unroll
    for (int e = 0; e < VE; ++e)
#pragma unroll
        for (int j = 0; j < K; ++j)
            w[j][e] = p.w_f32 ? reinterpret_cast<const float *>(p.w)[(c0 + e) * K + j]
                              : (float)reinterpret_cast<const E *>(p.w)[(c0 + e) * K + j];

    int seq = 0;
    int64_t bos = 0, eos = 0;                // no segment located yet
    auto locate = [&](int64_t t) __attribute__((always_inline)) {
        if (p.cu && p.n_seqs == 0) {
            bos = eos = 0;                   // no segments: every token is outside
        } else if (p.cu) {
            seq = seg_at(p.cu, p.n_seqs, p.n_tokens, t);
            bos = clamp_tok(p.cu[seq], p.n_tokens);
            eos = clamp_tok(p.cu[seq + 1], p.n_tokens);
        } else {
            seq = (int)(t / p.T);
            bos = (int64_t)seq * p.T;
            eos = bos + p.T;
        }
    };
    // window: win[j] = input at t - (K - 1) + j, j < K - 1 (filled only for bos <= t)
    U win[K > 1 ? K - 1 : 1];
    auto fill = [&](int64_t t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
            const int64_t pos = t - (K - 1) + j;
            if (pos >= bos) win[j].load(x + pos * p.D + c0);
            else if (st) win[j].load(st + ((int64_t)seq * K + (K + (pos - bos))) * p.D + c0);
            else win[j].zero();
        }
    };
    // one token: y[t] from the window and x[t], then the window moves on
    auto step = [&](int64_t t, const typename U::V &xv) __attribute__((always_inline)) {
        U cur;
#pragma unroll
        for (int e = 0; e < VE; ++e) cur.f[e] = (float)xv[e];
        typename U::V out;
#pragma unroll
        for (int e = 0; e < VE; ++e) {
            float acc = w[K - 1][e] * cur.f[e];
#pragma unroll
            for (int j = 0; j < K - 1; ++j) acc += w[j][e] * win[j].f[e];
            float r = (float)(E)acc;                         // the convolution's output in E
            if (p.silu) r = (float)(E)(r * sigmoidf_(r));
            out[e] = (E)r;
        }
        __builtin_nontemporal_store(out, reinterpret_cast<typename U::V *>(y + t * p.D + c0));
#pragma unroll
        for (int j = 0; j + 1 < K - 1; ++j) win[j] = win[j + 1];
        if constexpr (K > 1) win[K - 2] = cur;
    };
    locate(t0);
    if (bos <= t0 && t0 + RUN <= eos && t0 + RUN <= p.n_tokens) {
        // the whole run inside one segment: every row in flight at once, then the math
        fill(t0);
        typename U::V rows[RUN];
        unroll<RUN>([&](auto i) __attribute__((always_inline)) {
            rows[i] = *reinterpret_cast<const typename U::V *>(x + (t0 + i) * p.D + c0);
        });
        unroll<RUN>([&](auto i) __attribute__((always_inline)) { step(t0 + i, rows[i]); });
        return;
    }
    // a run that meets a segment boundary or the end of the tokens: token by token
    const int64_t t1 = t0 + RUN < p.n_tokens ? t0 + RUN : p.n_tokens;
    if (bos <= t0 && t0 < eos) fill(t0);
#pragma unroll 1
    for (int64_t t = t0; t < t1; ++t) {
        if (t > t0 && t >= eos) {            // the run enters the next packed segment(s)
            locate(t);
            if (bos <= t && t < eos) fill(t);
        }
        if (t < bos || t >= eos) {           // a token outside every segment (a malformed table)
            *reinterpret_cast<typename U::V *>(y + t * p.D + c0) = typename U::V{};
            continue;
        }
        step(t, *reinterpret_cast<const typename U::V *>(x + t * p.D + c0));
    }
}

// final conv cache of each sequence: the last K inputs of (initial cache, x[bos..eos));
// a thread reads all K units of its (sequence, channel unit) before writing any, so
// state_out may be state_in
template <typename E, int K>
__global__ void __launch_bounds__(256) conv_state_kernel(const ConvParams p) {
    using U = Unit<E>;
    constexpr int VE = U::VE;
    typedef typename U::V V;
    const int64_t ncg = p.D / VE;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (int64_t)p.n_seqs * ncg) return;
    const int seq = (int)(gid / ncg);
    const int64_t c0 = (gid % ncg) * VE;
    int64_t bos, eos;
    if (p.cu) {
        bos = clamp_tok(p.cu[seq], p.n_tokens);
        eos = clamp_tok(p.cu[seq + 1], p.n_tokens);
        if (eos < bos) eos = bos;
    } else {
        bos = (int64_t)seq * p.T;
        eos = bos + p.T;
    }
    const E *x = reinterpret_cast<const E *>(p.x);
    const E *st = reinterpret_cast<const E *>(p.state_in);
    V v[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const int64_t pos = eos - K + j;
        if (pos >= bos) v[j] = *reinterpret_cast<const V *>(x + pos * p.D + c0);
        else if (st) v[j] = *reinterpret_cast<const V *>(st + ((int64_t)seq * K + (K + (pos - bos))) * p.D + c0);
        else v[j] = V{};
    }
    E *so = reinterpret_cast<E *>(p.state_out);
#pragma unroll
    for (int j = 0; j < K; ++j) *reinterpret_cast<V *>(so + ((int64_t)seq * K + j) * p.D + c0) = v[j];
}

template <typename E, int K>
static hipError_t conv_k(const ConvParams &p, hipStream_t stream) {
    constexpr int VE = 16 / (int)sizeof(E);
    const int64_t ncg = p.D / VE;
    const int64_t runs = (p.n_tokens + RUN - 1) / RUN;
    const int64_t threads = runs * ncg;
    if (threads > 0)
        hipLaunchKernelGGL((causal_conv_kernel<E, K>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                           p);
    if (p.state_out && p.n_seqs > 0) {
        const int64_t st = (int64_t)p.n_seqs * ncg;
        hipLaunchKernelGGL((conv_state_kernel<E, K>), dim3((unsigned)((st + 255) / 256)), dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

template <typename E>
static hipError_t conv_t(const ConvParams &p, hipStream_t stream) {
    switch (p.K) {
        case 1: return conv_k<E, 1>(p, stream);
        case 2: return conv_k<E, 2>(p, stream);
        case 3: return conv_k<E, 3>(p, stream);
        case 4: return conv_k<E, 4>(p, stream);
        case 5: return conv_k<E, 5>(p, stream);
        case 6: return conv_k<E, 6>(p, stream);
        case 7: return conv_k<E, 7>(p, stream);
        case 8: return conv_k<E, 8>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t causal_conv(int dtype, const ConvParams &p, hipStream_t stream) {
    if (dtype == 1) return conv_t<__bf16>(p, stream);
    if (dtype == 2) return conv_t<_Float16>(p, stream);
    return conv_t<float>(p, stream);
}

}  // namespace vgdr

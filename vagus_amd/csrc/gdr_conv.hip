// The layer's short causal convolution + SiLU over a whole call's tokens
// (ShortConv, opt.py:15-100; fla's causal_conv1d as the reference calls it,
// :73-77), for prefill.  The decode kernel applies the same convolution per
// token; here it is one HBM pass over x.
//
// A thread owns VE = 16 / sizeof(E) consecutive channels (one 16-byte unit)
// for a run of RUN = 8 consecutive tokens.  A workgroup holds 16 units x 16
// consecutive runs, so a wavefront reads 16 neighbouring units (256 bytes) of
// four token rows per load.  The run's K - 1 + RUN input rows are all
// loaded before any arithmetic and kept as loaded (16-bit values unconverted),
// which keeps a thread within 128 VGPRs and so the whole grid of a 340M-shaped
// projection (B8 T4096 D1024: 4096 waves) resident at once.  Each input unit is
// loaded once per run plus K - 1 times at the run's start (those hit in cache).
// Inputs before a sequence's first token come from its conv cache [K, D] (the
// previous call's last K inputs, linear_attention.py:929-941) or are zero; a run
// that crosses into the next packed segment goes token by token and restarts its
// window there.  Measured at that shape: RUN 16 (occupancy 3) 25.2 us, RUN 8
// 23.2 us, RUN 4 26.7 us with one run of all 128 units per 128 threads; RUN 8
// with 16 x 16 workgroups 22.6 us (32 x 8: 23.2, 8 x 32: 22.9, 4 x 64: 33.9);
// a plain copy of the same bytes 22.2 us.
#include <type_traits>

#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

namespace {

constexpr int RUN = 8;
constexpr int CG_PER_GROUP = 16;

// channel units (16 bytes each) per workgroup of the prefill conv: CG_PER_GROUP,
// or all of them when there are fewer
__host__ __device__ __forceinline__ int conv_cg_per_group(int64_t ncg) {
    return ncg < CG_PER_GROUP ? (int)ncg : CG_PER_GROUP;
}

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

// the segment holding token t: its index and token range (dense: sequences of T
// tokens; packed: the cu_seqlens entry, clamped; no segments: an empty range)
struct Seg {
    int seq;
    int64_t bos, eos;
};
__device__ __forceinline__ Seg seg_of(const ConvParams &p, int64_t t) {
    if (p.cu && p.n_seqs == 0) return Seg{0, 0, 0};
    if (p.cu) {
        const int s = seg_at(p.cu, p.n_seqs, p.n_tokens, t);
        return Seg{s, clamp_tok(p.cu[s], p.n_tokens), clamp_tok(p.cu[s + 1], p.n_tokens)};
    }
    // (32-bit division where the tokens allow it: a 64-bit one is a long VALU sequence
    // ahead of every load of the run)
    const int s = p.n_tokens <= 0x7fffffff ? (int)((uint32_t)t / (uint32_t)p.T) : (int)(t / p.T);
    return Seg{s, (int64_t)s * p.T, (int64_t)s * p.T + p.T};
}

}  // namespace

// WT: the weights' type (fp32 or E); WV: the weights are 16-byte aligned, so a
// thread's VE x K block (contiguous, 16 * K or 32 * K bytes) is read with 16-byte loads
template <typename E, typename WT, int K, bool WV>
__global__ void __launch_bounds__(256) causal_conv_kernel(const ConvParams p) {
    constexpr int VE = 16 / (int)sizeof(E);
    typedef E V __attribute__((ext_vector_type(VE)));
    const int64_t ncg = p.D / VE;
    // A workgroup covers 256 / CG_PER_GROUP consecutive runs of CG_PER_GROUP channel
    // units (of all of them when there are fewer): a run's K - 1 window rows are the previous run's last rows, read
    // by a thread of the same workgroup (so from this CU's cache) except for the
    // workgroup's first run.  (With one run per 128 channel units, consecutive runs sat
    // in consecutive workgroups, on different XCDs, and about half of the window rows
    // were fetched from HBM a second time.)
    const int cgw = conv_cg_per_group(ncg), rpw = 256 / cgw;
    const int tid = threadIdx.x;
    if (tid >= cgw * rpw) return;
    const uint32_t ncb = (uint32_t)((ncg + cgw - 1) / cgw);
    const int64_t cg = (int64_t)(blockIdx.x % ncb) * cgw + tid % cgw;
    const int64_t run = (int64_t)(blockIdx.x / ncb) * rpw + tid / cgw;
    const int64_t t0 = run * RUN;
    if (cg >= ncg || t0 >= p.n_tokens) return;
    const int64_t c0 = cg * VE;
    const E *x = reinterpret_cast<const E *>(p.x);
    const E *st = reinterpret_cast<const E *>(p.state_in);
    E *y = reinterpret_cast<E *>(p.y);

    // weights w[c][j] of channels c0..c0+VE-1 as loaded: wb[e * K + j]
    WT wb[VE * K];
    const WT *wsrc = reinterpret_cast<const WT *>(p.w) + c0 * K;
    if constexpr (WV) {
        typedef uint32_t U4 __attribute__((ext_vector_type(4)));
        constexpr int N16 = VE * K * (int)sizeof(WT) / 16;
        static_assert(VE * K * (int)sizeof(WT) % 16 == 0, "weight block");
        unroll<N16>([&](auto i) __attribute__((always_inline)) {
            const U4 u = reinterpret_cast<const U4 *>(wsrc)[decltype(i)::value];
            __builtin_memcpy(reinterpret_cast<char *>(wb) + 16 * decltype(i)::value, &u, 16);
        });
    } else {
        unroll<VE * K>([&](auto i) __attribute__((always_inline)) { wb[i] = wsrc[decltype(i)::value]; });
    }

    // the input row at pos of segment sg (pos < bos: its cache, or zeros).  Branch-free:
    // the load is from x, the cache or (for zeros) row bos of x, and the zeros are
    // selected afterwards; a branch around each load would make the wave wait for it
    // where the branches join.
    auto row = [&](const Seg &sg, int64_t pos) __attribute__((always_inline)) -> V {
        const bool in = pos >= sg.bos;
        const E *src = in   ? x + pos * p.D + c0
                       : st ? st + ((int64_t)sg.seq * K + (K + (pos - sg.bos))) * p.D + c0
                            : x + sg.bos * p.D + c0;
        const V v = *reinterpret_cast<const V *>(src);
        return in || st ? v : V{};
    };
    // y[t] from the K rows win[0..K-1] = inputs t - K + 1 .. t
    auto out = [&](int64_t t, const V *win) __attribute__((always_inline)) {
        V o;
#pragma unroll
        for (int e = 0; e < VE; ++e) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < K; ++j) acc += (float)wb[e * K + j] * (float)win[j][e];
            float r = (float)(E)acc;                         // the convolution's output in E
            if (p.silu) r = (float)(E)(r * sigmoidf_(r));
            o[e] = (E)r;
        }
        __builtin_nontemporal_store(o, reinterpret_cast<V *>(y + t * p.D + c0));
    };
    const Seg sg = seg_of(p, t0);
    if (sg.bos <= t0 && t0 + RUN <= sg.eos && t0 + RUN <= p.n_tokens) {
        // the whole run inside one segment: every row in flight at once, then the math
        V rows[K - 1 + RUN];
        unroll<K - 1>([&](auto j) __attribute__((always_inline)) { rows[j] = row(sg, t0 - (K - 1) + j); });
        unroll<RUN>([&](auto i) __attribute__((always_inline)) {
            rows[K - 1 + i] = *reinterpret_cast<const V *>(x + (t0 + i) * p.D + c0);
        });
        // (the scheduler would otherwise interleave the arithmetic with the loads and
        // issue the last rows only after the first ones arrived)
        __builtin_amdgcn_sched_barrier(0);
        unroll<RUN>([&](auto i) __attribute__((always_inline)) { out(t0 + i, rows + decltype(i)::value); });
        return;
    }
    // a run that meets a segment boundary or the end of the tokens: token by token,
    // win[] sliding
    const int64_t t1 = t0 + RUN < p.n_tokens ? t0 + RUN : p.n_tokens;
    Seg cur = sg;
    V win[K];
    auto fill = [&](int64_t t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) win[j] = row(cur, t - (K - 1) + j);
    };
    if (cur.bos <= t0 && t0 < cur.eos) fill(t0);
#pragma unroll 1
    for (int64_t t = t0; t < t1; ++t) {
        if (t > t0 && t >= cur.eos) {        // the run enters the next packed segment(s)
            cur = seg_of(p, t);
            if (cur.bos <= t && t < cur.eos) fill(t);
        }
        if (t < cur.bos || t >= cur.eos) {   // a token outside every segment (a malformed table)
            *reinterpret_cast<V *>(y + t * p.D + c0) = V{};
            continue;
        }
        win[K - 1] = *reinterpret_cast<const V *>(x + t * p.D + c0);
        out(t, win);
#pragma unroll
        for (int j = 0; j < K - 1; ++j) win[j] = win[j + 1];
    }
}

// final conv cache of each sequence: the last K inputs of (initial cache, x[bos..eos));
// a thread reads all K units of its (sequence, channel unit) before writing any, so
// state_out may be state_in
template <typename E, int K>
__global__ void __launch_bounds__(256) conv_state_kernel(const ConvParams p) {
    constexpr int VE = 16 / (int)sizeof(E);
    typedef E V __attribute__((ext_vector_type(VE)));
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
    if (runs > 0 && ncg > 0) {
        const int cgw = conv_cg_per_group(ncg), rpw = 256 / cgw;
        const int64_t groups = (ncg + cgw - 1) / cgw * ((runs + rpw - 1) / rpw);
        if (groups > 0x7fffffff) return hipErrorInvalidValue;
        const dim3 grid((unsigned)groups);
        const bool wv = ((uintptr_t)p.w & 15) == 0;
        if (p.w_f32 && !std::is_same<E, float>::value) {
            if (wv) hipLaunchKernelGGL((causal_conv_kernel<E, float, K, true>), grid, dim3(256), 0, stream, p);
            else hipLaunchKernelGGL((causal_conv_kernel<E, float, K, false>), grid, dim3(256), 0, stream, p);
        } else {
            if (wv) hipLaunchKernelGGL((causal_conv_kernel<E, E, K, true>), grid, dim3(256), 0, stream, p);
            else hipLaunchKernelGGL((causal_conv_kernel<E, E, K, false>), grid, dim3(256), 0, stream, p);
        }
    }
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

// Token-by-token gated delta rule (the decode step at T = 1) for gfx950.
//
// One workgroup of 256 threads owns one (sequence, head) and keeps the whole
// fp32 state S[DK][DV] in registers for the length of its token range.  Thread
// (row group rg, column group cg) holds rows rg + NRG*i (i < RPT) of the four
// columns 4cg..4cg+3, so each state load / store is one coalesced 16-byte
// access and a wavefront covers whole contiguous rows.  Per token
// (linear_attention.py:176-193):
//     S' = Diag(a) S                                  (a = exp(g): scalar or per row)
//     kS = k^T S',  qS = q^T S',  qk = q . k          one pass, one reduction
//     u  = beta (v - kS)   (v without the delta rule)
//     o  = scale (qS + qk u)                          = scale q^T (S' + k u^T)
//     S  = S' + k u^T
// so S is read once and written once per call regardless of T.  The state
// streams through once per call, so it is read and written non-temporally
// (measured: 30.7 -> 25.5 us per decode step at B=64 H=16 dk=dv=128).
#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

// Producer of one channel with the short conv: SiLU(sum_j w[c][j] x[t - K + 1 + j][c])
// for the token t of a sequence starting at bos; x is [n_tokens, HD] (HD = H * d), the
// cache [K, HD] holds the sequence's K inputs before bos.  The convolution's and the
// SiLU's results are rounded to E, as the module computes them in its dtype.  At the
// sequence's last token (last = true) the K inputs just read are exactly the cache's
// next contents, and are written back to it here: the owner thread of a channel is
// its only reader, and it has read its last old value in this call.
template <typename E>
__device__ __forceinline__ float conv_silu(const E *x, E *cache, const void *w, int w_f32, int64_t HD, int64_t c,
                                           int K, int64_t t, int64_t bos, bool last) {
    using EL = Elem<E>;
    // c passes through an empty asm: the weight loads then stay in the token step
    // instead of being hoisted out of the token loop into registers held across it
    asm volatile("" : "+v"(c));
    // all K (<= 8) input and weight loads are issued together (predicated), not one
    // dependent load per tap
    E xs[8];
    float wt[8];
    unroll<8>([&](auto j) __attribute__((always_inline)) {
        xs[j] = EL::from_f(0.f);
        wt[j] = 0.f;
        if (j < K) {
            const int64_t pos = t - (K - 1) + j;
            xs[j] = pos >= bos ? x[pos * HD + c] : cache[(K + (pos - bos)) * HD + c];
            wt[j] = w_f32 ? reinterpret_cast<const float *>(w)[c * K + j]
                          : EL::to_f(reinterpret_cast<const E *>(w)[c * K + j]);
        }
    });
    float acc = 0.f;
    unroll<8>([&](auto j) __attribute__((always_inline)) { acc += wt[j] * EL::to_f(xs[j]); });
    if (last) {
        unroll<8>([&](auto j) __attribute__((always_inline)) {
            if (j < K) cache[(int64_t)j * HD + c] = xs[j];
        });
    }
    const float y = EL::to_f(EL::from_f(acc));
    return EL::to_f(EL::from_f(y * sigmoidf_(y)));
}

// MODE bit 0: the output epilogue; bit 1: the short conv; bit 2: an explicit
// write vector w_t in place of beta_t k_t (the asymmetric delta rule,
// linear_attention.py:161-170, :185-188).  All are template choices: as
// run-time branches they add registers to every variant (the GDN kernel fills
// the chip in one pass only within 128 VGPRs).
template <int DK, int DV, typename E, int GATE, int MODE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GATE == 2 || (MODE & 4) ? 1 : 4)))
recurrent_kernel(const RecParams p) {
    constexpr bool EPI = MODE & 1, CONV = MODE & 2, WR = MODE & 4;
    constexpr int NT = 256;
    constexpr int NCG = DV / 4;             // column groups (float4 each)
    constexpr int NRG = NT / NCG;           // row groups
    constexpr int RPT = DK / NRG;           // rows per thread
    constexpr int NWV = NT / 64;
    static_assert(NT % NCG == 0 && DK % NRG == 0 && 64 % NCG == 0, "thread layout");
    using EL = Elem<E>;

    __shared__ __attribute__((aligned(16))) float qs[DK];
    __shared__ __attribute__((aligned(16))) float ks[DK];
    __shared__ __attribute__((aligned(16))) float vs[DV];
    __shared__ __attribute__((aligned(16))) float gv[GATE == 2 ? DK : 1];
    __shared__ __attribute__((aligned(16))) float red[NWV][2][DV];
    __shared__ float redqk[NWV];
    __shared__ float nrm[NWV][2];           // fused L2 norm: per-wave sums of q^2, k^2
    __shared__ float sc[2];                 // decay (scalar gate), beta
    __shared__ __attribute__((aligned(16))) float wsv[WR ? DK : 4];    // the write vector w_t
    __shared__ __attribute__((aligned(16))) float gts[EPI ? DV : 4];   // epilogue: output gate of the token
    __shared__ __attribute__((aligned(16))) float gms[EPI ? DV : 4];   // epilogue: RMSNorm weight

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = tid % NCG, rg = tid / NCG;
    const int h = blockIdx.x % p.H;
    const int seq = blockIdx.x / p.H;
    int64_t bos, eos;
    if (p.cu) {
        int64_t a = p.cu[seq], b = p.cu[seq + 1];
        a = a < 0 ? 0 : (a > p.n_tokens ? p.n_tokens : a);
        b = b < a ? a : (b > p.n_tokens ? p.n_tokens : b);
        bos = a;
        eos = b;
    } else {
        bos = (int64_t)seq * p.T;
        eos = bos + p.T;
    }
    const E *qg = reinterpret_cast<const E *>(p.q);
    const E *kg = reinterpret_cast<const E *>(p.k);
    const E *vg = reinterpret_cast<const E *>(p.v);
    E *og = reinterpret_cast<E *>(p.o);
    const int H = p.H;

    if constexpr (EPI) {
        for (int i = tid; i < DV; i += NT)
            gms[i] = p.ep.gamma_f32 ? reinterpret_cast<const float *>(p.ep.gamma)[i]
                                    : EL::to_f(reinterpret_cast<const E *>(p.ep.gamma)[i]);
    }

    const int64_t sbase = ((int64_t)seq * H + h) * DK * DV;
    f32x4 S[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
        S[i] = p.h0 ? __builtin_nontemporal_load(
                          reinterpret_cast<const f32x4 *>(p.h0 + sbase + (int64_t)(rg + NRG * i) * DV + 4 * cg))
                    : f32x4{0.f, 0.f, 0.f, 0.f};

    for (int64_t t = bos; t < eos; ++t) {
        // token operands -> LDS (fp32); thread i < DK owns q_i, k_i (and g_i)
        const int64_t qo = (t * H + h) * DK, vo = (t * H + h) * DV;
        const bool own = tid < DK;
        float qv, kv;
        if constexpr (CONV) {
            // fused short conv + SiLU of the q, k projections (linear_attention.py:741-745, :929-941)
            const int64_t HDK = (int64_t)H * DK, c = (int64_t)h * DK + tid, cb = (int64_t)seq * p.cv.K * HDK;
            const bool last = t == eos - 1;
            qv = own ? conv_silu<E>(qg, reinterpret_cast<E *>(p.cv.cq) + cb, p.cv.wq, p.cv.w_f32, HDK, c, p.cv.K, t,
                                    bos, last)
                     : 0.f;
            kv = own ? conv_silu<E>(kg, reinterpret_cast<E *>(p.cv.ck) + cb, p.cv.wk, p.cv.w_f32, HDK, c, p.cv.K, t,
                                    bos, last)
                     : 0.f;
        } else {
            qv = own ? EL::to_f(qg[qo + tid]) : 0.f;
            kv = own ? EL::to_f(kg[qo + tid]) : 0.f;
        }
        if (p.fz.qk_l2norm) {
            // fused producer (linear_attention.py:703-706): x rsqrt(sum x^2 + 1e-6), rounded to E
            float sq = qv * qv, sk = kv * kv;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                sq += __shfl_xor(sq, off);
                sk += __shfl_xor(sk, off);
            }
            if (lane == 0) {
                nrm[wave][0] = sq;
                nrm[wave][1] = sk;
            }
            __syncthreads();
            sq = sk = 0.f;
#pragma unroll
            for (int w = 0; w < NWV; ++w) {
                sq += nrm[w][0];
                sk += nrm[w][1];
            }
            qv = EL::to_f(EL::from_f(qv * rsqrtf(sq + 1e-6f)));
            kv = EL::to_f(EL::from_f(kv * rsqrtf(sk + 1e-6f)));
        }
        if (own) {
            qs[tid] = qv * p.scale;
            ks[tid] = kv;
            if constexpr (WR) wsv[tid] = EL::to_f(reinterpret_cast<const E *>(p.w)[qo + tid]);
            if constexpr (GATE == 2) {
                float gl;
                if (p.fz.gate_act) {                       // fused gate activation from the pre-activation f
                    const float f = p.fz.gate_16 ? EL::to_f(reinterpret_cast<const E *>(p.g)[qo + tid]) : p.g[qo + tid];
                    gl = gate_activation(f, p.fz.A_log[h], p.fz.dt_bias[(int64_t)h * DK + tid], p.fz.lb_set, p.fz.lb);
                } else {
                    gl = p.g[qo + tid];
                }
                gv[tid] = __expf(gl);
            }
        }
        for (int i = tid; i < DV; i += NT) {
            if constexpr (CONV) {
                const int64_t HDV = (int64_t)H * DV;
                vs[i] = conv_silu<E>(vg, reinterpret_cast<E *>(p.cv.cv) + (int64_t)seq * p.cv.K * HDV, p.cv.wv,
                                     p.cv.w_f32, HDV, (int64_t)h * DV + i, p.cv.K, t, bos, t == eos - 1);
            } else {
                vs[i] = EL::to_f(vg[vo + i]);
            }
            if constexpr (EPI) gts[i] = EL::to_f(reinterpret_cast<const E *>(p.ep.gate)[vo + i]);
        }
        if (tid == 0) {
            sc[0] = (GATE == 1 && p.g) ? __expf(p.g[t * H + h]) : 1.f;
            const float b = (!WR && p.use_delta) ? p.beta[t * H + h] : 0.f;     // beta may be NULL with w
            sc[1] = WR ? 1.f : (p.use_delta && p.fz.beta_sigmoid ? sigmoidf_(b) : b);   // w carries the strength
        }
        __syncthreads();

        f32x4 kS = {0.f, 0.f, 0.f, 0.f}, qS = {0.f, 0.f, 0.f, 0.f};
        float qk = 0.f;
        const float a0 = sc[0];
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int r = rg + NRG * i;
            const float a = (GATE == 2) ? gv[r] : a0;
            S[i] *= a;
            kS += ks[r] * S[i];
            qS += qs[r] * S[i];
            qk += qs[r] * (WR ? wsv[r] : ks[r]);
        }
        // reduce over the row groups of this wave (lanes NCG apart share columns)
#pragma unroll
        for (int off = NCG; off < 64; off <<= 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kS[e] += __shfl_xor(kS[e], off);
                qS[e] += __shfl_xor(qS[e], off);
            }
            qk += __shfl_xor(qk, off);
        }
        if (lane < NCG) {
            st4(&red[wave][0][4 * cg], kS);
            st4(&red[wave][1][4 * cg], qS);
        }
        if (lane == 0) redqk[wave] = qk;
        __syncthreads();
        kS = ld4(&red[0][0][4 * cg]);
        qS = ld4(&red[0][1][4 * cg]);
        qk = redqk[0];
#pragma unroll
        for (int w = 1; w < NWV; ++w) {
            kS += ld4(&red[w][0][4 * cg]);
            qS += ld4(&red[w][1][4 * cg]);
            qk += redqk[w];
        }
        const f32x4 v4 = ld4(&vs[4 * cg]);
        const f32x4 u = p.use_delta ? sc[1] * (v4 - kS) : v4;
        const f32x4 o = qS + qk * u;                     // q was pre-scaled
        if constexpr (EPI) {
            // the layer's output epilogue (linear_attention.py:814-825) on the row this
            // workgroup holds: x = o in E, out = x rsqrt(mean x^2 + eps) gamma silu(gate).
            // Wave 0 holds every column (lanes cg of each NCG-lane group).
            if (wave == 0) {
                // the gate and gamma were staged in LDS with v (loads issued early, no
                // registers held across the step)
                float x[4], ss = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[e] = EL::to_f(EL::from_f(o[e]));
                    ss += x[e] * x[e];
                }
#pragma unroll
                for (int m = 1; m < NCG; m <<= 1) ss += __shfl_xor(ss, m);
                const float r = rsqrtf(ss * (1.f / DV) + p.ep.eps);
                if (rg == 0) {
                    const f32x4 gt = ld4(&gts[4 * cg]), gm = ld4(&gms[4 * cg]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        og[vo + 4 * cg + e] = EL::from_f(x[e] * r * gm[e] * (gt[e] * sigmoidf_(gt[e])));
                }
            }
        } else if (rg == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) og[vo + 4 * cg + e] = EL::from_f(o[e]);
        }
#pragma unroll
        for (int i = 0; i < RPT; ++i) S[i] += (WR ? wsv[rg + NRG * i] : ks[rg + NRG * i]) * u;
        __syncthreads();                                 // LDS reused by the next token
    }

    if (p.ht) {
#pragma unroll
        for (int i = 0; i < RPT; ++i)
            __builtin_nontemporal_store(S[i], reinterpret_cast<f32x4 *>(p.ht + sbase + (int64_t)(rg + NRG * i) * DV + 4 * cg));
    }
    // (the conv caches were advanced in the last token's step; an empty segment leaves
    // its cache as it was)
}

template <int DK, int DV, typename E, int GATE>
static hipError_t launch_rec(const RecParams &p, hipStream_t stream) {
    const int64_t blocks = (int64_t)p.n_seqs * p.H;
    if (blocks == 0) return hipSuccess;
    const int mode = (p.ep.gate ? 1 : 0) | (p.cv.K ? 2 : 0) | (p.w ? 4 : 0);
#define VGDR_REC(M)                                                                                           \
    case M:                                                                                                    \
        hipLaunchKernelGGL((recurrent_kernel<DK, DV, E, GATE, M>), dim3((unsigned)blocks), dim3(256), 0, stream, p); \
        break;
    switch (mode) { VGDR_REC(0) VGDR_REC(1) VGDR_REC(2) VGDR_REC(3) VGDR_REC(4) VGDR_REC(5) VGDR_REC(6) VGDR_REC(7) }
#undef VGDR_REC
    return hipGetLastError();
}

template <int DK, int DV, typename E>
static hipError_t rec_gate(int gate_vector, const RecParams &p, hipStream_t s) {
    return gate_vector ? launch_rec<DK, DV, E, 2>(p, s) : launch_rec<DK, DV, E, 1>(p, s);
}

template <typename E>
static hipError_t rec_shape(int dk, int dv, int gate_vector, const RecParams &p, hipStream_t s) {
    if (dk == 64) return dv == 64 ? rec_gate<64, 64, E>(gate_vector, p, s) : rec_gate<64, 128, E>(gate_vector, p, s);
    return dv == 64 ? rec_gate<128, 64, E>(gate_vector, p, s) : rec_gate<128, 128, E>(gate_vector, p, s);
}

hipError_t recurrent_fwd(int dtype, int dk, int dv, int gate_vector, const RecParams &p,
                         hipStream_t stream) {
    if (dtype == 1) return rec_shape<__bf16>(dk, dv, gate_vector, p, stream);
    if (dtype == 2) return rec_shape<_Float16>(dk, dv, gate_vector, p, stream);
    return rec_shape<float>(dk, dv, gate_vector, p, stream);
}

// ---------------------------------------------------------------------------
// packed-batch schedule: lens, chunk counts, chunk offsets, longest-first order
// ---------------------------------------------------------------------------
__device__ inline int64_t seg_len(const int32_t *cu, int n, int64_t n_tokens) {
    int64_t a = cu[n], b = cu[n + 1];
    a = a < 0 ? 0 : (a > n_tokens ? n_tokens : a);
    b = b < a ? a : (b > n_tokens ? n_tokens : b);
    return b - a;
}

__global__ void __launch_bounds__(256) varlen_rank_kernel(const int32_t *cu, int n_seqs, int64_t n_tokens,
                                                          int chunk, int32_t *ws, int sort) {
    const int s = blockIdx.x * 256 + threadIdx.x;
    if (s >= n_seqs) return;
    int32_t *lens = ws, *chunks = ws + n_seqs, *order = ws + 3 * n_seqs + 1;
    const int64_t L = seg_len(cu, s, n_tokens);
    lens[s] = (int32_t)L;
    chunks[s] = (int32_t)((L + chunk - 1) / chunk);
    if (!sort) {
        order[s] = s;
        return;
    }
    int rank = 0;
    for (int t = 0; t < n_seqs; ++t) {
        const int64_t Lt = seg_len(cu, t, n_tokens);
        rank += (Lt > L) || (Lt == L && t < s);
    }
    order[rank] = s;
}

// exclusive prefix sum of chunks -> chunk_offsets[0..n_seqs], one workgroup
__global__ void __launch_bounds__(1024) varlen_offsets_kernel(int n_seqs, int32_t *ws) {
    __shared__ int64_t part[1024];
    const int32_t *chunks = ws + n_seqs;
    int32_t *offs = ws + 2 * n_seqs;
    const int tid = threadIdx.x;
    const int per = (n_seqs + 1023) / 1024;
    const int lo = tid * per, hi = lo + per < n_seqs ? lo + per : n_seqs;
    int64_t sum = 0;
    for (int i = lo; i < hi; ++i) sum += chunks[i];
    part[tid] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {        // Hillis-Steele inclusive scan
        const int64_t x = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += x;
        __syncthreads();
    }
    int64_t run = tid ? part[tid - 1] : 0;
    for (int i = lo; i < hi; ++i) {
        offs[i] = (int32_t)run;
        run += chunks[i];
    }
    if (tid == 1023) offs[n_seqs] = (int32_t)part[1023];
}

hipError_t varlen_prepare(const int32_t *cu, int n_seqs, int64_t n_tokens, int chunk, int32_t *ws,
                          hipStream_t stream) {
    if (n_seqs <= 0) return hipSuccess;
    const int sort = n_seqs <= 16384;                 // O(n^2) ranking; beyond that index order
    hipLaunchKernelGGL(varlen_rank_kernel, dim3((n_seqs + 255) / 256), dim3(256), 0, stream, cu, n_seqs,
                       n_tokens, chunk, ws, sort);
    hipLaunchKernelGGL(varlen_offsets_kernel, dim3(1), dim3(1024), 0, stream, n_seqs, ws);
    return hipGetLastError();
}

}  // namespace vgdr

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
#include <type_traits>

#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

// an element of type E from its bits (a 16-bit type zero-extended into 32 bits)
template <typename E>
__device__ __forceinline__ float bits_to_f(uint32_t b) {
    if constexpr (sizeof(E) == 2) return Elem<E>::to_f(__builtin_bit_cast(E, (uint16_t)b));
    else return __uint_as_float(b);
}

// One channel of the four-tap short conv for one token of the decode step:
// SiLU(sum_j w[c][j] x[t - 3 + j][c]) for the token t = bos of a sequence, x
// [n_tokens, HD] (HD = H * d), the cache [4, HD] holding the sequence's 4 inputs
// before bos.  load() only issues the loads (the taps, and the channel's weight row
// as one aligned vector of WT), so that the caller decides what is in flight beside
// them; apply() then does the arithmetic.  Loaded values are kept as loaded: a
// conversion at load time would make the divergent owner branch wait for its loads
// where it ends.  The convolution's and the SiLU's results are rounded to E, as the
// module computes them in its dtype.  The 4 inputs read are exactly the cache's next
// contents, and apply() writes them back: the owner thread of a channel is its only
// reader, and it has read its last old value.
template <typename E, typename WT>
struct ConvTaps {
    using EL = Elem<E>;
    typedef WT WV __attribute__((ext_vector_type(4)));
    E xs[4];
    WV w4;
    // x: the token's input row at x[t * LD]; the cache rows [K, HD]
    __device__ __forceinline__ void load(const E *x, const E *cache, const void *w, int64_t HD, int64_t LD,
                                         int64_t c, int64_t t) {
        unroll<4>([&](auto j) __attribute__((always_inline)) {
            xs[j] = j == 3 ? x[t * LD + c] : cache[(int64_t)(j + 1) * HD + c];
        });
        w4 = reinterpret_cast<const WV *>(w)[c];
    }
    __device__ __forceinline__ float apply(E *cache, int64_t HD, int64_t c) const {
        float acc = 0.f;
        unroll<4>([&](auto j) __attribute__((always_inline)) {
            acc += (float)w4[decltype(j)::value] * EL::to_f(xs[j]);
        });
        // the cache row addresses are rebuilt here rather than kept from load()
        asm volatile("" : "+v"(c));
        unroll<4>([&](auto j) __attribute__((always_inline)) { cache[(int64_t)j * HD + c] = xs[j]; });
        const float y = EL::to_f(EL::from_f(acc));
        return EL::to_f(EL::from_f(y * sigmoidf_(y)));
    }
};

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

// The layer's decode step with the short conv (GatedDeltaNet.decode_step at L = 1,
// linear_attention.py:918-952): one token per sequence, four conv taps with 16-byte
// aligned weights of type WT (E or fp32), a state to read.  MODE: the EPI and WR bits
// of recurrent_kernel (the conv is implied).  The layout is recurrent_kernel's; the
// order of the work differs:
//   * the state's loads are issued first thing (buffer loads: one lane offset for all
//     rows), then the token's operand loads;
//   * the producers (conv, SiLU, L2 norm, q . k) run on threads 0..dk-1 and stage
//     their results in LDS behind barriers that order LDS only;
//   * the state is read as loaded: the dot products take the decay from the staged
//     q and k (per channel) or as one factor after the sum (scalar), and the update
//     S <- diag(a) S + k u^T is one FMA per element.
// Measured at B64 H16 dk=dv=128, bf16, 24 rotating layers: 29.2 us with the
// producers waiting for the state (recurrent_kernel), 26.4 us with the operand
// loads ahead of the state's, 25.7 us in this order before the decay folding.  A
// producer wave of its own (5 waves per workgroup) needs more than 96 VGPRs and
// spills: 31 us.
// dv = 256 (the reference's dk 128 / dv 256 mixer heads) runs 512 threads with
// another layout: wave w owns columns 32 w .. 32 w + 31 of every row (lane (rg,
// cg): rows rg + 8 i, columns 32 w + 4 cg .. + 3), so a thread's share of the
// 128 KiB state is 64 fp32 registers and kS, qS are reduced inside the wave.
// No barrier then separates a wave's state loads from its state stores: waves
// whose rows arrive first update and store them while the others still load.
// With one workgroup per CU (B64 H4), a layout whose reduction spans the waves
// made every wave of the chip load, then every wave store (58 % of HBM).
template <int DV> constexpr int decode_threads() { return DV > 128 ? 512 : 256; }

// torch's softplus at beta 1, threshold 20, with the accurate expf / log1pf
__device__ __forceinline__ float softplus_acc(float x) { return x > 20.f ? x : log1pf(expf(x)); }

template <int DK, int DV, typename E, int GATE, int MODE, typename WT>
__global__ void __launch_bounds__(decode_threads<DV>())
__attribute__((amdgpu_waves_per_eu(GATE == 2 || (MODE & 4) || DV > 128 ? 1 : 4)))
decode_conv_kernel(const RecParams p) {
    constexpr bool EPI = MODE & 1, WR = MODE & 4;
    constexpr bool WIDE = DV > 128;                             // one wave per 32 columns
    constexpr int NT = decode_threads<DV>();
    constexpr int NCG = WIDE ? 8 : DV / 4;                      // column groups (WIDE: per wave)
    constexpr int NRG = WIDE ? 8 : NT / NCG;                    // row groups (WIDE: per wave)
    constexpr int RPT = DK / NRG;
    constexpr int NWV = NT / 64;
    constexpr int K = 4;
    static_assert(WIDE ? (NWV * 32 == DV && DK % NRG == 0 && DK <= NT)
                       : (NT % NCG == 0 && DK % NRG == 0 && 64 % NCG == 0 && DK <= NT && DV <= NT), "thread layout");
    using EL = Elem<E>;

    // qs, ks: q (scaled) and k, times the per-channel decay with GATE 2; kr: k itself
    __shared__ __attribute__((aligned(16))) float qs[DK];
    __shared__ __attribute__((aligned(16))) float ks[DK];
    __shared__ __attribute__((aligned(16))) float kr[GATE == 2 ? DK : 1];
    __shared__ __attribute__((aligned(16))) float vs[DV];
    __shared__ __attribute__((aligned(16))) float gv[GATE == 2 ? DK : 1];
    __shared__ __attribute__((aligned(16))) float red[WIDE ? 1 : NWV][2][WIDE ? 4 : DV];
    __shared__ float nrm[NWV][3];           // per-wave sums: q^2, k^2, then q . k (q . w)
    __shared__ float ssq[WIDE ? NWV : 1];   // WIDE epilogue: per-wave sums of o^2
    __shared__ float gpart[GATE == 1 ? NWV : 1][2];   // per-wave sums of W_a x, W_b x (gate projections)
    __shared__ float sc[2];                 // decay (scalar gate), beta
    __shared__ __attribute__((aligned(16))) float wsv[WR ? DK : 4];
    __shared__ __attribute__((aligned(16))) float gts[EPI ? DV : 4];
    __shared__ __attribute__((aligned(16))) float gms[EPI ? DV : 4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // cg: the thread's column group (columns 4 cg .. + 3); rg: its first row
    const int cg = WIDE ? NCG * wave + (lane & (NCG - 1)) : tid % NCG;
    const int rg = WIDE ? lane / NCG : tid / NCG;
    const int H = p.H;
    const int h = blockIdx.x % H;
    const int seq = blockIdx.x / H;
    const int64_t t = seq;                  // one token per sequence
    const int64_t qo = (t * H + h) * DK, vo = (t * H + h) * DV;
    const int64_t sbase = ((int64_t)seq * H + h) * DK * DV;
    const bool own = tid < DK, vown = tid < DV;
    E *og = reinterpret_cast<E *>(p.o);

    // (1) the state
    const __amdgpu_buffer_rsrc_t s_in = buffer_rsrc(p.h0 + sbase, DK * DV * 4);
    const uint32_t so = (uint32_t)(rg * DV + 4 * cg) * 4;
    // dv = 128 (several workgroups per CU) issues the state first; WIDE (one
    // workgroup per CU) issues it after the token's operands, so that the conv,
    // norm and gate work below waits for those alone and runs while the state
    // arrives (measured at B64 H4: 15.5 -> 15.0 us)
    f32x4 S[RPT];
    if constexpr (!WIDE) {
#pragma unroll
        for (int i = 0; i < RPT; ++i) S[i] = buffer_load_nt4(s_in, so, (uint32_t)(NRG * i * DV * 4));
    }

    // (2) the token's operands
    const int64_t HDK = (int64_t)H * DK, HDV = (int64_t)H * DV;
    const int64_t LDQ = p.ld_qk ? p.ld_qk : HDK, LDV = p.ld_v ? p.ld_v : HDV;   // input token rows
    const int64_t cq = (int64_t)h * DK + tid, cvc = (int64_t)h * DV + tid;
    E *cache_q = reinterpret_cast<E *>(p.cv.cq) + (int64_t)seq * K * HDK;
    E *cache_k = reinterpret_cast<E *>(p.cv.ck) + (int64_t)seq * K * HDK;
    E *cache_v = reinterpret_cast<E *>(p.cv.cv) + (int64_t)seq * K * HDV;
    ConvTaps<E, WT> tq, tk, tv;
    E wr = EL::from_f(0.f), gtr = EL::from_f(0.f);
    uint32_t gr = 0;
    float gsc = 0.f, bsc = 0.f, gmv = 0.f;
    if (own) {
        tq.load(reinterpret_cast<const E *>(p.q), cache_q, p.cv.wq, HDK, LDQ, cq, t);
        tk.load(reinterpret_cast<const E *>(p.k), cache_k, p.cv.wk, HDK, LDQ, cq, t);
        if constexpr (WR) wr = reinterpret_cast<const E *>(p.w)[qo + tid];
        if constexpr (GATE == 2)
            gr = p.fz.gate_act && p.fz.gate_16 && sizeof(E) == 2
                     ? (uint32_t)reinterpret_cast<const uint16_t *>(p.g)[qo + tid]
                     : reinterpret_cast<const uint32_t *>(p.g)[qo + tid];
    }
    if (vown) {
        tv.load(reinterpret_cast<const E *>(p.v), cache_v, p.cv.wv, HDV, LDV, cvc, t);
        if constexpr (EPI) {
            gtr = reinterpret_cast<const E *>(p.ep.gate)[t * LDV + cvc];
            gmv = p.ep.gamma_f32 ? reinterpret_cast<const float *>(p.ep.gamma)[tid]
                                 : EL::to_f(reinterpret_cast<const E *>(p.ep.gamma)[tid]);
        }
    }
    // the gate projections W_a[h] . x and W_b[h] . x (GateProj): every thread up
    // to GU 16-byte slices of the row, loaded with the token's other operands and
    // summed after the conv (dim <= GU NT VE, checked by the API)
    const bool gproj = GATE == 1 && p.gp.x != nullptr;
    constexpr int GVE = 16 / (int)sizeof(E), GU = 2;
    typedef E GV __attribute__((ext_vector_type(GVE)));
    GV gxv[GU], gav[GU], gbv[GU];
    if (gproj) {
        const int nu = p.gp.dim / GVE;
        const E *xr = reinterpret_cast<const E *>(p.gp.x) + t * (int64_t)p.gp.dim;
        const E *wa = reinterpret_cast<const E *>(p.gp.w) + (int64_t)h * p.gp.dim;
        const E *wb = wa + (int64_t)H * p.gp.dim;
        const bool wbeta = !WR && p.use_delta;
#pragma unroll
        for (int i = 0; i < GU; ++i) {
            const int u = tid + i * NT;
            gxv[i] = gav[i] = gbv[i] = GV{};
            if (u < nu) {
                gxv[i] = *reinterpret_cast<const GV *>(xr + (int64_t)u * GVE);
                gav[i] = *reinterpret_cast<const GV *>(wa + (int64_t)u * GVE);
                if (wbeta) gbv[i] = *reinterpret_cast<const GV *>(wb + (int64_t)u * GVE);
            }
        }
    } else if (tid == 0) {
        if (GATE == 1 && p.g) gsc = p.g[t * H + h];
        if (!WR && p.use_delta) bsc = p.beta[t * H + h];
    }

    if constexpr (WIDE) {
#pragma unroll
        for (int i = 0; i < RPT; ++i) S[i] = buffer_load_nt4(s_in, so, (uint32_t)(NRG * i * DV * 4));
    }
    // (3) producers: conv + SiLU (linear_attention.py:741-745) advancing the caches
    // (:929-941), the L2 norm (:703-706), q . k
    float qv = 0.f, kv = 0.f;
    if (own) {
        qv = tq.apply(cache_q, HDK, cq);
        kv = tk.apply(cache_k, HDK, cq);
    }
    if (gproj) {
        float pa = 0.f, pb = 0.f;
#pragma unroll
        for (int i = 0; i < GU; ++i)
#pragma unroll
            for (int e = 0; e < GVE; ++e) {
                pa += (float)gxv[i][e] * (float)gav[i][e];
                pb += (float)gxv[i][e] * (float)gbv[i][e];
            }
        pa = wave_sum64(pa);
        pb = wave_sum64(pb);
        if (lane == 0) {
            gpart[wave][0] = pa;
            gpart[wave][1] = pb;
        }
        if (!p.fz.qk_l2norm) lds_barrier();                  // else the norm's barrier below
    }
    if (p.fz.qk_l2norm) {
        float sq = wave_sum64(qv * qv), sk = wave_sum64(kv * kv);
        if (lane == 0) {
            nrm[wave][0] = sq;
            nrm[wave][1] = sk;
        }
        lds_barrier();
        sq = sk = 0.f;
#pragma unroll
        for (int w = 0; w < NWV; ++w) {
            sq += nrm[w][0];
            sk += nrm[w][1];
        }
        qv = EL::to_f(EL::from_f(qv * rsqrtf(sq + 1e-6f)));
        kv = EL::to_f(EL::from_f(kv * rsqrtf(sk + 1e-6f)));
    }
    qv *= p.scale;
    {
        float qk = qv * (WR ? EL::to_f(wr) : kv);
        qk = wave_sum64(qk);
        if (lane == 0) nrm[wave][2] = qk;
    }
    if (own) {
        float a = 1.f;
        if constexpr (GATE == 2) {
            const float gf = p.fz.gate_act && p.fz.gate_16 ? bits_to_f<E>(gr) : __uint_as_float(gr);
            const float gl = p.fz.gate_act ? gate_activation(gf, p.fz.A_log[h], p.fz.dt_bias[(int64_t)h * DK + tid],
                                                             p.fz.lb_set, p.fz.lb)
                                           : gf;
            a = __expf(gl);
            gv[tid] = a;
            kr[tid] = kv;
        }
        qs[tid] = qv * a;
        ks[tid] = kv * a;
        if constexpr (WR) wsv[tid] = EL::to_f(wr);
    }
    if (vown) {
        vs[tid] = tv.apply(cache_v, HDV, cvc);
        if constexpr (EPI) {
            gts[tid] = EL::to_f(gtr);
            gms[tid] = gmv;
        }
    }
    if (tid == 0) {
        if (gproj) {
            float sa = 0.f, sb = 0.f;
#pragma unroll
            for (int w = 0; w < NWV; ++w) {
                sa += gpart[w][0];
                sb += gpart[w][1];
            }
            // nn.Linear's outputs in the element type, then the gate (fp32)
            gsc = p.gp.neg_a[h] * softplus_acc(EL::to_f(EL::from_f(sa)) + p.gp.dt_bias[h]);
            bsc = EL::to_f(EL::from_f(sb));
        }
        sc[0] = (GATE == 1 && (p.g || gproj)) ? __expf(gsc) : 1.f;
        sc[1] = WR ? 1.f : (p.use_delta && p.fz.beta_sigmoid ? sigmoidf_(bsc) : bsc);
    }
    lds_barrier();

    // (4) the state math on the state as loaded
    f32x4 kS = {0.f, 0.f, 0.f, 0.f}, qS = {0.f, 0.f, 0.f, 0.f};
    const float a0 = sc[0];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int r = rg + NRG * i;
        kS += ks[r] * S[i];
        qS += qs[r] * S[i];
    }
    if constexpr (GATE != 2) {
        kS *= a0;
        qS *= a0;
    }
    // the sums over the row groups: lanes l ^ NCG .. l ^ 32 (WIDE: all of them)
#pragma unroll
    for (int off = NCG; off < 64; off <<= 1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (off == 8) {                                    // lanes l ^ 8: the other half of the row
                kS[e] += dpp_f<0x128>(kS[e]);
                qS[e] += dpp_f<0x128>(qS[e]);
            } else {
                kS[e] += __shfl_xor(kS[e], off);
                qS[e] += __shfl_xor(qS[e], off);
            }
        }
    }
    float qk = nrm[0][2];
#pragma unroll
    for (int w = 1; w < NWV; ++w) qk += nrm[w][2];
    if constexpr (!WIDE) {
        // ... and over the waves
        if (lane < NCG) {
            st4(&red[wave][0][4 * cg], kS);
            st4(&red[wave][1][4 * cg], qS);
        }
        lds_barrier();
        kS = ld4(&red[0][0][4 * cg]);
        qS = ld4(&red[0][1][4 * cg]);
#pragma unroll
        for (int w = 1; w < NWV; ++w) {
            kS += ld4(&red[w][0][4 * cg]);
            qS += ld4(&red[w][1][4 * cg]);
        }
    }
    const f32x4 v4 = ld4(&vs[4 * cg]);
    const f32x4 u = p.use_delta ? sc[1] * (v4 - kS) : v4;
    const f32x4 o = qS + qk * u;                     // o = q^T (diag(a) S + k u^T)
    if constexpr (WIDE) {
        // the state first: its stores leave before the epilogue's barrier
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int r = rg + NRG * i;
            const float a = GATE == 2 ? gv[r] : a0;
            S[i] = a * S[i] + (WR ? wsv[r] : GATE == 2 ? kr[r] : ks[r]) * u;
        }
        if (p.ht) {
            const __amdgpu_buffer_rsrc_t s_out = buffer_rsrc(p.ht + sbase, DK * DV * 4);
#pragma unroll
            for (int i = 0; i < RPT; ++i) buffer_store_nt4(S[i], s_out, so, (uint32_t)(NRG * i * DV * 4));
        }
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = EL::to_f(EL::from_f(o[e]));
        if constexpr (EPI) {
            // the output epilogue (linear_attention.py:814-825): the row's sum of
            // squares over the wave's 32 columns (lanes 0 .. NCG - 1 hold them;
            // every row group has a copy), then over the waves
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += x[e] * x[e];
#pragma unroll
            for (int m = 1; m < NCG; m <<= 1) ss += __shfl_xor(ss, m);
            if (lane == 0) ssq[wave] = ss;
            lds_barrier();
            ss = 0.f;
#pragma unroll
            for (int w = 0; w < NWV; ++w) ss += ssq[w];
            const float r = rsqrtf(ss * (1.f / DV) + p.ep.eps);
            if (rg == 0) {
                const f32x4 gt = ld4(&gts[4 * cg]), gm = ld4(&gms[4 * cg]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    og[vo + 4 * cg + e] = EL::from_f(x[e] * r * gm[e] * (gt[e] * sigmoidf_(gt[e])));
            }
        } else if (rg == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) og[vo + 4 * cg + e] = EL::from_f(x[e]);
        }
        return;
    }
    if constexpr (EPI) {
        // the output epilogue (linear_attention.py:814-825); wave 0 holds every column
        if (wave == 0) {
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
    for (int i = 0; i < RPT; ++i) {
        const int r = rg + NRG * i;
        const float a = GATE == 2 ? gv[r] : a0;
        S[i] = a * S[i] + (WR ? wsv[r] : GATE == 2 ? kr[r] : ks[r]) * u;
    }
    if (p.ht) {
        const __amdgpu_buffer_rsrc_t s_out = buffer_rsrc(p.ht + sbase, DK * DV * 4);
#pragma unroll
        for (int i = 0; i < RPT; ++i) buffer_store_nt4(S[i], s_out, so, (uint32_t)(NRG * i * DV * 4));
    }
}

template <int DK, int DV, typename E, int GATE>
static hipError_t launch_rec(const RecParams &p, hipStream_t stream) {
    const int64_t blocks = (int64_t)p.n_seqs * p.H;
    if (blocks == 0) return hipSuccess;
    // the layer's decode step (one token per sequence, a state, the conv's usual four
    // taps with 16-byte aligned weights) has its own kernel
    const bool aligned = (((uintptr_t)p.cv.wq | (uintptr_t)p.cv.wk | (uintptr_t)p.cv.wv) & 15) == 0;
    if (!p.cu && p.T == 1 && p.h0 && p.cv.K == 4 && aligned) {
        const int m = (p.ep.gate ? 1 : 0) | (p.w ? 4 : 0);
        const bool wf = p.cv.w_f32 && !std::is_same<E, float>::value;     // fp32 weights beside 16-bit inputs
#define VGDR_DEC(M)                                                                                           \
    case M:                                                                                                    \
        if (wf)                                                                                                \
            hipLaunchKernelGGL((decode_conv_kernel<DK, DV, E, GATE, M, float>), dim3((unsigned)blocks), dim3(256), 0, \
                               stream, p);                                                                     \
        else                                                                                                   \
            hipLaunchKernelGGL((decode_conv_kernel<DK, DV, E, GATE, M, E>), dim3((unsigned)blocks), dim3(256), 0,  \
                               stream, p);                                                                     \
        break;
        switch (m) { VGDR_DEC(0) VGDR_DEC(1) VGDR_DEC(4) VGDR_DEC(5) }
#undef VGDR_DEC
        return hipGetLastError();
    }
    const int mode = (p.ep.gate ? 1 : 0) | (p.cv.K ? 2 : 0) | (p.w ? 4 : 0);
#define VGDR_REC(M)                                                                                           \
    case M:                                                                                                    \
        hipLaunchKernelGGL((recurrent_kernel<DK, DV, E, GATE, M>), dim3((unsigned)blocks), dim3(256), 0, stream, p); \
        break;
    switch (mode) { VGDR_REC(0) VGDR_REC(1) VGDR_REC(2) VGDR_REC(3) VGDR_REC(4) VGDR_REC(5) VGDR_REC(6) VGDR_REC(7) }
#undef VGDR_REC
    return hipGetLastError();
}

template <int DK, int DV, typename E, int GATE>
static hipError_t launch_dec_wide(const RecParams &p, hipStream_t stream) {
    // dv = 256: the one-token decode step with the short conv only (the API refuses
    // every other call at this width)
    const int64_t blocks = (int64_t)p.n_seqs * p.H;
    if (blocks == 0) return hipSuccess;
    const bool aligned = (((uintptr_t)p.cv.wq | (uintptr_t)p.cv.wk | (uintptr_t)p.cv.wv) & 15) == 0;
    if (p.cu || p.T != 1 || !p.h0 || p.cv.K != 4 || !aligned || p.w) return hipErrorInvalidValue;
    const bool wf = p.cv.w_f32 && !std::is_same<E, float>::value;
    const dim3 grid((unsigned)blocks), block(decode_threads<DV>());
    if (p.ep.gate) {
        if (wf) hipLaunchKernelGGL((decode_conv_kernel<DK, DV, E, GATE, 1, float>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((decode_conv_kernel<DK, DV, E, GATE, 1, E>), grid, block, 0, stream, p);
    } else {
        if (wf) hipLaunchKernelGGL((decode_conv_kernel<DK, DV, E, GATE, 0, float>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((decode_conv_kernel<DK, DV, E, GATE, 0, E>), grid, block, 0, stream, p);
    }
    return hipGetLastError();
}

template <int DK, int DV, typename E>
static hipError_t rec_gate(int gate_vector, const RecParams &p, hipStream_t s) {
    if constexpr (DV > 128)
        return gate_vector ? launch_dec_wide<DK, DV, E, 2>(p, s) : launch_dec_wide<DK, DV, E, 1>(p, s);
    else
        return gate_vector ? launch_rec<DK, DV, E, 2>(p, s) : launch_rec<DK, DV, E, 1>(p, s);
}

template <typename E>
static hipError_t rec_shape(int dk, int dv, int gate_vector, const RecParams &p, hipStream_t s) {
    if (dv == 256) return dk == 64 ? rec_gate<64, 256, E>(gate_vector, p, s) : rec_gate<128, 256, E>(gate_vector, p, s);
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

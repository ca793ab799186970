// Fused chunkwise prefill of the gated delta rule (GDN scalar gate, KDA
// per-channel gate, optional delta rule) for gfx950.
//
// One workgroup owns one (sequence, head, 16*NW-column dv tile) and walks the
// sequence chunk by chunk.  Wave w owns the 16 dv columns [16w, 16w+16) of the
// tile and keeps their fp32 state S[0:DK, cols] in MFMA accumulators (C
// layout, DK/16 tiles) for the whole sequence: the state chain
//     U~ = U - W S,   o = (Q*G) S + A U~,   S <- Gc (.) S + (K*Gend)^T U~
// runs register-to-register, with no LDS round trip and no barrier.
// The chunk-local, state-independent operands (K K^T and Q K^T gated and
// masked, T = (I + M)^-1, W = T diag(beta) (K*G)) are built cooperatively in
// LDS once per chunk.  Math: linear_attention.py:237-309 (scalar) and
// :312-425 (per-channel gate), in its unified per-channel form
//     M_ij = beta_i <k_i, k_j>_g (j < i),   A_ij = scale <q_i, k_j>_g (j <= i)
//     T = (I + M)^-1,  W = T diag(beta) (K*G),  U = T diag(beta) V
// where <x_i, y_j>_g = sum_c x_i[c] y_j[c] exp(gamma_i[c] - gamma_j[c]) and
// gamma is the in-chunk cumulative log decay (a scalar per token for GDN).
//
// Per-channel gates reach the MFMA through a sub-block factorisation:
// for token blocks I >= J of 16 and reference row r = 16 I,
//     exp(gamma_i - gamma_j) = exp(gamma_i - gamma_r) * exp(gamma_r - gamma_j)
// Off-diagonal blocks (j < r <= i) have both exponents <= 0.  A diagonal
// block's second factor is >= 1, bounded by the block's own decay range; a
// block whose range exceeds Elem<E>::gate_range nats takes an exact pairwise
// path instead (never forming an overflowing exponential).
#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

template <int DK, int CH, int NW, typename E, int GATE>
struct ChunkLayout {
    static constexpr int NT = 64 * NW;                // threads
    static constexpr int DVT = 16 * NW;               // dv columns per workgroup
    static constexpr int NB = CH / 16;                // token blocks per chunk
    static constexpr int NKB = DK / 16;               // key blocks
    static constexpr int PK = DK + Elem<E>::pad;      // pitch of [CH][DK] E arrays
    static constexpr int PC = CH + Elem<E>::pad;      // pitch of [*][CH] E arrays
    static constexpr int PV = DVT + Elem<E>::pad;     // pitch of the staged V rows
    static constexpr int PF = CH + 4;                 // pitch of [CH][CH] fp32 arrays
    static constexpr int PG = DK + 4;                 // pitch of the per-channel gamma table
    static constexpr int ES = sizeof(E);

    static constexpr int szKs = CH * PK * ES;
    static constexpr int szKsT = DK * PC * ES;
    static constexpr int szVsT = DVT * PC * ES;
    static constexpr int szAqk = CH * PC * ES;
    static constexpr int szMW = cmax(CH * PF * 4, CH * PK * ES);              // M, then W
    static constexpr int szT = CH * PF * 4;
    static constexpr int szTT = cmax(cmax(CH * PF * 4, CH * PC * ES), CH * PV * ES);  // V rows, TT, then TE
    static constexpr int szGam = (GATE == 2 ? CH * PG : CH) * 4;

    static constexpr int oKs = 0;
    static constexpr int oQs = oKs + szKs;
    static constexpr int oKsT = oQs + szKs;
    static constexpr int oVsT = oKsT + szKsT;
    static constexpr int oAqk = oVsT + szVsT;
    static constexpr int oMW = oAqk + szAqk;
    static constexpr int oT = oMW + szMW;
    static constexpr int oTT = oT + szT;
    static constexpr int oGam = oTT + szTT;
    static constexpr int oBeta = oGam + szGam;
    static constexpr int oG = oBeta + CH * 4;         // scalar gate: G_i = exp(gamma_i)
    static constexpr int oGend = oG + CH * 4;         // scalar gate: exp(gamma_C - gamma_i)
    static constexpr int oGc = oGend + CH * 4;        // exp(gamma_C): DK values (vector) / 1
    static constexpr int oFlag = oGc + DK * 4;        // diag-block pairwise flags
    static constexpr int BYTES = oFlag + 16;
    static_assert(BYTES <= 160 * 1024, "LDS budget exceeded");
    static_assert(oQs % 16 == 0 && oKsT % 16 == 0 && oVsT % 16 == 0 && oAqk % 16 == 0 &&
                      oMW % 16 == 0 && oT % 16 == 0 && oTT % 16 == 0 && oGam % 16 == 0,
                  "LDS arrays must stay 16-byte aligned");
};

// Copy rows [0, CH) x cols [0, NCOL) of a token-major global matrix into LDS
// (row pitch P), zero-filling rows >= valid_rows and columns >= valid_cols.
// Global row t starts at src + t * stride.  All loads are issued before any
// store so their latencies overlap.
template <typename E, int CH, int NCOL, int P, int NT>
__device__ inline void load_rows(E *dst, const E *src, int64_t stride, int valid_rows,
                                 int valid_cols, int tid) {
    constexpr int VE = 16 / sizeof(E);                // elements per 16-byte vector
    constexpr int VPR = NCOL / VE;                    // vectors per row
    constexpr int NV = CH * VPR;
    static_assert(NCOL % VE == 0 && NV % NT == 0, "tile does not split evenly");
    constexpr int PER = NV / NT;
    Vec16 r[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int vi = tid + i * NT;
        const int row = vi / VPR, col = (vi % VPR) * VE;
        if (row < valid_rows && col < valid_cols)
            r[i] = *reinterpret_cast<const Vec16 *>(src + (int64_t)row * stride + col);
        else
            r[i] = Vec16{{0u, 0u, 0u, 0u}};
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int vi = tid + i * NT;
        const int row = vi / VPR, col = (vi % VPR) * VE;
        uint32_t *d = reinterpret_cast<uint32_t *>(dst + row * P + col);
        // 8-byte stores: the padded pitch keeps rows 8- but not 16-byte aligned
        reinterpret_cast<uint2 *>(d)[0] = uint2{r[i].w[0], r[i].w[1]};
        reinterpret_cast<uint2 *>(d)[1] = uint2{r[i].w[2], r[i].w[3]};
    }
}

template <int DK, int CH, int NW, typename E, int GATE>
__global__ void __launch_bounds__(64 * NW, 1) chunk_fwd_kernel(const ChunkParams p) {
    using L = ChunkLayout<DK, CH, NW, E, GATE>;
    using EL = Elem<E>;
    using F = typename EL::frag;
    constexpr int NT = L::NT, NB = L::NB, NKB = L::NKB, DVT = L::DVT;
    constexpr int PK = L::PK, PC = L::PC, PF = L::PF, PG = L::PG, PV = L::PV;

    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    E *Ks = reinterpret_cast<E *>(smem + L::oKs);
    E *Qs = reinterpret_cast<E *>(smem + L::oQs);
    E *KsT = reinterpret_cast<E *>(smem + L::oKsT);
    E *VsT = reinterpret_cast<E *>(smem + L::oVsT);
    E *Aqk = reinterpret_cast<E *>(smem + L::oAqk);
    float *Mf = reinterpret_cast<float *>(smem + L::oMW);
    E *Ws = reinterpret_cast<E *>(smem + L::oMW);
    float *Tf = reinterpret_cast<float *>(smem + L::oT);
    float *TTf = reinterpret_cast<float *>(smem + L::oTT);
    E *TE = reinterpret_cast<E *>(smem + L::oTT);
    E *Vrow = reinterpret_cast<E *>(smem + L::oTT);
    float *gam = reinterpret_cast<float *>(smem + L::oGam);
    float *bet = reinterpret_cast<float *>(smem + L::oBeta);
    float *Gs = reinterpret_cast<float *>(smem + L::oG);
    float *Gend = reinterpret_cast<float *>(smem + L::oGend);
    float *Gc = reinterpret_cast<float *>(smem + L::oGc);
    int *flag = reinterpret_cast<int *>(smem + L::oFlag);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;

    // ---- work item --------------------------------------------------------
    const int tile = blockIdx.x % p.n_tiles;
    const int unit = blockIdx.x / p.n_tiles;
    const int h = unit % p.H;
    const int pos = unit / p.H;
    const int seq = p.order ? p.order[pos] : pos;
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
    const int H = p.H, DV = p.DV;
    const int col0 = tile * DVT;
    const int wcol = col0 + 16 * wave;               // this wave's first dv column
    const bool wvalid = wcol < DV;                   // DV % 16 == 0
    const E *qg = reinterpret_cast<const E *>(p.q);
    const E *kg = reinterpret_cast<const E *>(p.k);
    const E *vg = reinterpret_cast<const E *>(p.v);
    E *og = reinterpret_cast<E *>(p.o);
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * DV;

    // ---- entry state (C layout: S[kt][j] = S[16kt + 4g + j][wcol + r16]) ---
    f32x4 S[NKB];
    const int64_t sbase = ((int64_t)seq * H + h) * DK * DV;
#pragma unroll
    for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            S[kt][j] = (p.h0 && wvalid) ? p.h0[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV + wcol + r16]
                                        : 0.f;

    const int64_t len = eos - bos;
    const int nchunks = (int)((len + CH - 1) / CH);
    for (int c = 0; c < nchunks; ++c) {
        const int64_t t0 = bos + (int64_t)c * CH;
        const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
        __syncthreads();                              // previous chunk's LDS readers are done

        // ---- L1: chunk inputs -> LDS ----------------------------------------
        load_rows<E, CH, DK, PK, NT>(Ks, kg + t0 * sqk + (int64_t)h * DK, sqk, clen, DK, tid);
        load_rows<E, CH, DK, PK, NT>(Qs, qg + t0 * sqk + (int64_t)h * DK, sqk, clen, DK, tid);
        load_rows<E, CH, DVT, PV, NT>(Vrow, vg + t0 * sv + (int64_t)h * DV + col0, sv, clen,
                                      DV - col0, tid);
        if constexpr (GATE == 2) {
            constexpr int NV = CH * DK / 4;
            static_assert(NV % NT == 0, "gate tile does not split evenly");
            f32x4 r[NV / NT];
#pragma unroll
            for (int i = 0; i < NV / NT; ++i) {
                const int vi = tid + i * NT, row = vi / (DK / 4), col = (vi % (DK / 4)) * 4;
                r[i] = row < clen ? ld4(p.g + ((t0 + row) * H + h) * DK + col) : f32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < NV / NT; ++i) {
                const int vi = tid + i * NT, row = vi / (DK / 4), col = (vi % (DK / 4)) * 4;
                st4(gam + row * PG + col, r[i]);
            }
        } else {
            if (tid < CH) gam[tid] = (p.g && tid < clen) ? p.g[(t0 + tid) * H + h] : 0.f;
        }
        if (tid < CH) bet[tid] = (p.use_delta && tid < clen) ? p.beta[(t0 + tid) * H + h] : 0.f;
        __syncthreads();

        // ---- L1b: transposes, cumulative decay --------------------------------
        // KsT[c][t..t+3] = Ks[t..t+3][c];  VsT[n][t..t+3] = Vrow[t..t+3][n]
        for (int it = tid; it < DK * (CH / 4); it += NT) {
            const int cc = it % DK, t = (it / DK) * 4;
            F x = {Ks[(t + 0) * PK + cc], Ks[(t + 1) * PK + cc], Ks[(t + 2) * PK + cc],
                   Ks[(t + 3) * PK + cc]};
            st_frag<E>(KsT + cc * PC + t, x);
        }
        for (int it = tid; it < DVT * (CH / 4); it += NT) {
            const int n = it % DVT, t = (it / DVT) * 4;
            F x = {Vrow[(t + 0) * PV + n], Vrow[(t + 1) * PV + n], Vrow[(t + 2) * PV + n],
                   Vrow[(t + 3) * PV + n]};
            st_frag<E>(VsT + n * PC + t, x);
        }
        if constexpr (GATE == 2) {
            // per-channel inclusive scan over CH tokens: NP parts of CH/NP tokens
            constexpr int NP = NT / DK;
            constexpr int SEG = CH / NP;
            static_assert(NP >= 1 && CH % NP == 0, "scan split");
            const int cc = tid % DK, part = tid / DK;
            if (part < NP) {
                float acc = 0.f;
                for (int t = part * SEG; t < (part + 1) * SEG; ++t) {
                    acc += gam[t * PG + cc];
                    gam[t * PG + cc] = acc;
                }
            }
            __syncthreads();
            float off = 0.f;                          // totals of the earlier parts, read
            if (part < NP)                            // before any part is updated
                for (int q2 = 0; q2 < part; ++q2) off += gam[((q2 + 1) * SEG - 1) * PG + cc];
            if (tid < NB) flag[tid] = 0;
            __syncthreads();
            if (part < NP && part > 0)
                for (int t = part * SEG; t < (part + 1) * SEG; ++t) gam[t * PG + cc] += off;
            __syncthreads();
            if (tid < DK) Gc[tid] = __expf(gam[(CH - 1) * PG + tid]);
            // diagonal sub-block decay ranges -> pairwise fallback flags
            for (int it = tid; it < NB * DK; it += NT) {
                const int b = it / DK, cc2 = it % DK;
                const float range = gam[(16 * b) * PG + cc2] - gam[(16 * b + 15) * PG + cc2];
                if (range > EL::gate_range) flag[b] = 1;          // benign race: all write 1
            }
        } else {
            if (wave == 0) {
                float x = gam[lane < CH ? lane : CH - 1];
                if (lane >= CH) x = 0.f;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const float y = __shfl_up(x, o);
                    if (lane >= o) x += y;
                }
                const float last = __shfl(x, CH - 1);
                if (lane < CH) {
                    gam[lane] = x;
                    Gs[lane] = __expf(x);
                    Gend[lane] = __expf(last - x);
                }
                if (lane == 0) Gc[0] = __expf(last);
            }
        }
        __syncthreads();

        // ---- L3: gated K K^T (-> M) and Q K^T (-> Aqk), lower blocks ---------
        // Job (I, J, which) computes X = K_J Y_I^T (Y = K or Q), so that the C
        // layout holds X[4g + jj][r] = <y_i, k_j> with i = 16I + r, j = 16J + 4g + jj:
        // four consecutive j of one row i, stored with one vector write.
        {
            constexpr int NL = NB * (NB + 1) / 2;
            const int njobs = p.use_delta ? 2 * NL : NL;
            for (int job = wave; job < njobs; job += NW) {
                const bool isq = job < NL;           // Q jobs first (always present)
                int tI = isq ? job : job - NL;
                int I = 0;
                while (tI > I) { tI -= I + 1; ++I; }
                const int J = tI;
                const E *Ys = isq ? Qs : Ks;
                const int i_tok = 16 * I + r16;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                bool pairwise = false;
                if constexpr (GATE == 2) pairwise = (I == J) && flag[I];
                if (!pairwise) {
                    if constexpr (GATE == 2) {
                        const int rr = 16 * I;
                        acc = contract(acc, NKB,
                            [&](int kb) {     // A: k_j * exp(gamma_r - gamma_j)
                                const int cc = 16 * kb + 4 * g4, jt = 16 * J + r16;
                                f32x4 x = EL::tof(ld_frag<E>(Ks + jt * PK + cc));
                                f32x4 e = exp4(ld4(gam + rr * PG + cc) - ld4(gam + jt * PG + cc));
                                return EL::cvt(x * e);
                            },
                            [&](int kb) {     // B: y_i * exp(gamma_i - gamma_r)
                                const int cc = 16 * kb + 4 * g4;
                                f32x4 x = EL::tof(ld_frag<E>(Ys + i_tok * PK + cc));
                                f32x4 e = exp4(ld4(gam + i_tok * PG + cc) - ld4(gam + rr * PG + cc));
                                return EL::cvt(x * e);
                            });
                    } else {
                        acc = contract(acc, NKB,
                            [&](int kb) { return ld_frag<E>(Ks + (16 * J + r16) * PK + 16 * kb + 4 * g4); },
                            [&](int kb) { return ld_frag<E>(Ys + i_tok * PK + 16 * kb + 4 * g4); });
                    }
                } else if constexpr (GATE == 2) {
                    // exact pairwise products for a diagonal block with a large decay range
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int j_tok = 16 * J + 4 * g4 + jj;
                        float s = 0.f;
                        if (j_tok <= i_tok) {
                            for (int cc = 0; cc < DK; cc += 4) {
                                f32x4 y = EL::tof(ld_frag<E>(Ys + i_tok * PK + cc));
                                f32x4 kx = EL::tof(ld_frag<E>(Ks + j_tok * PK + cc));
                                f32x4 e = exp4(ld4(gam + i_tok * PG + cc) - ld4(gam + j_tok * PG + cc));
                                f32x4 t4 = y * kx * e;
                                s += t4[0] + t4[1] + t4[2] + t4[3];
                            }
                        }
                        acc[jj] = s;
                    }
                }
                // epilogue: decay (scalar gate), beta / scale, masks
                f32x4 out;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j_tok = 16 * J + 4 * g4 + jj;
                    float d = 1.f;
                    if constexpr (GATE != 2) d = (j_tok <= i_tok) ? __expf(gam[i_tok] - gam[j_tok]) : 0.f;
                    const float x = acc[jj] * d;
                    out[jj] = isq ? ((j_tok <= i_tok) ? p.scale * x : 0.f)
                                  : ((j_tok < i_tok) ? bet[i_tok] * x : 0.f);
                }
                if (isq)
                    st_frag<E>(Aqk + i_tok * PC + 16 * J + 4 * g4, EL::cvt(out));
                else
                    st4(Mf + i_tok * PF + 16 * J + 4 * g4, out);
            }
        }
        __syncthreads();

        // Q -> scale * (Q * G) for the state read-out (raw Q no longer needed)
        for (int it = tid; it < CH * (DK / 4); it += NT) {
            const int t = it / (DK / 4), cc = (it % (DK / 4)) * 4;
            f32x4 x = EL::tof(ld_frag<E>(Qs + t * PK + cc));
            f32x4 gf;
            if constexpr (GATE == 2) gf = exp4(ld4(gam + t * PG + cc));
            else gf = f32x4{Gs[t], Gs[t], Gs[t], Gs[t]};
            st_frag<E>(Qs + t * PK + cc, EL::cvt(x * gf * p.scale));
        }

        if (p.use_delta) {
            // ---- L4: T = (I + M)^-1, diagonal 16x16 blocks by substitution ----
            if (wave == 0 && lane < 16 * NB) {
                const int b = lane >> 4, jc = lane & 15;
                float t[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float acc = (i == jc) ? 1.f : 0.f;
                    const float *mrow = Mf + (16 * b + i) * PF + 16 * b;
#pragma unroll
                    for (int m = 0; m < i; ++m) acc -= mrow[m] * t[m];
                    t[i] = acc;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) Tf[(16 * b + i) * PF + 16 * b + jc] = t[i];
#pragma unroll
                for (int i = 0; i < 16; i += 4)
                    st4(TTf + (16 * b + jc) * PF + 16 * b + i, f32x4{t[i], t[i + 1], t[i + 2], t[i + 3]});
            }
            __syncthreads();
            // off-diagonal blocks: T_IJ = -T_II sum_{K=J}^{I-1} M_IK T_KJ, by distance
#pragma unroll
            for (int dist = 1; dist < NB; ++dist) {
                for (int jb = wave; jb < NB - dist; jb += NW) {
                    const int J = jb, I = jb + dist;
                    f32x4 X = {0.f, 0.f, 0.f, 0.f};
                    for (int K = J; K < I; ++K)
                        X = mfma_kb1(ld4(Mf + (16 * I + r16) * PF + 16 * K + 4 * g4),
                                     ld4(TTf + (16 * J + r16) * PF + 16 * K + 4 * g4), X);
                    const f32x4 Y = mfma_kb1(ld4(Tf + (16 * I + r16) * PF + 16 * I + 4 * g4), X,
                                             f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int j = 0; j < 4; ++j) Tf[(16 * I + 4 * g4 + j) * PF + 16 * J + r16] = -Y[j];
                    st4(TTf + (16 * J + r16) * PF + 16 * I + 4 * g4, -Y);
                }
                __syncthreads();
            }
            // TE = T diag(beta) (lower triangle), in the element type.  TE overwrites
            // TT, which the barrier above retired.
            for (int it = tid; it < CH * (CH / 4); it += NT) {
                const int i = it / (CH / 4), j = (it % (CH / 4)) * 4;
                f32x4 t = ld4(Tf + i * PF + j) * ld4(bet + j);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j + e > i) t[e] = 0.f;
                st_frag<E>(TE + i * PC + j, EL::cvt(t));
            }
            // KsT -> (K * G)^T
            for (int it = tid; it < DK * (CH / 4); it += NT) {
                const int cc = it % DK, t = (it / DK) * 4;
                f32x4 x = EL::tof(ld_frag<E>(KsT + cc * PC + t));
                f32x4 gf;
                if constexpr (GATE == 2)
                    gf = exp4(f32x4{gam[(t + 0) * PG + cc], gam[(t + 1) * PG + cc],
                                    gam[(t + 2) * PG + cc], gam[(t + 3) * PG + cc]});
                else
                    gf = ld4(Gs + t);
                st_frag<E>(KsT + cc * PC + t, EL::cvt(x * gf));
            }
            __syncthreads();
            // ---- L6: W^T = (K*G)^T TE^T -> Ws (row-major W) --------------------
            for (int job = wave; job < NKB * NB; job += NW) {
                const int a = job % NKB, b = job / NKB;
                f32x4 acc = contract(f32x4{0.f, 0.f, 0.f, 0.f}, b + 1,
                    [&](int kb) { return ld_frag<E>(KsT + (16 * a + r16) * PC + 16 * kb + 4 * g4); },
                    [&](int kb) { return ld_frag<E>(TE + (16 * b + r16) * PC + 16 * kb + 4 * g4); });
                st_frag<E>(Ws + (16 * b + r16) * PK + 16 * a + 4 * g4, EL::cvt(acc));
            }
            __syncthreads();
        }
        // KsT -> (K * Gend)^T, rebuilt from the raw row-major K
        for (int it = tid; it < DK * (CH / 4); it += NT) {
            const int cc = it % DK, t = (it / DK) * 4;
            f32x4 x = {EL::to_f(Ks[(t + 0) * PK + cc]), EL::to_f(Ks[(t + 1) * PK + cc]),
                       EL::to_f(Ks[(t + 2) * PK + cc]), EL::to_f(Ks[(t + 3) * PK + cc])};
            f32x4 gf;
            if constexpr (GATE == 2) {
                const float last = gam[(CH - 1) * PG + cc];
                gf = exp4(f32x4{last - gam[(t + 0) * PG + cc], last - gam[(t + 1) * PG + cc],
                                last - gam[(t + 2) * PG + cc], last - gam[(t + 3) * PG + cc]});
            } else {
                gf = ld4(Gend + t);
            }
            st_frag<E>(KsT + cc * PC + t, EL::cvt(x * gf));
        }
        __syncthreads();

        // ---- S phase: this wave's 16 state columns, registers only -----------
        if (wvalid) {
            const E *Vw = VsT + (16 * wave + r16) * PC;      // this lane's V column
            f32x4 U[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                if (p.use_delta)
                    U[I] = contract(f32x4{0.f, 0.f, 0.f, 0.f}, I + 1,
                        [&](int kb) { return ld_frag<E>(TE + (16 * I + r16) * PC + 16 * kb + 4 * g4); },
                        [&](int kb) { return ld_frag<E>(Vw + 16 * kb + 4 * g4); });
                else
                    U[I] = EL::tof(ld_frag<E>(Vw + 16 * I + 4 * g4));
            }
            F Sb[NKB];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) Sb[kt] = EL::cvt(S[kt]);
            if (p.use_delta) {
#pragma unroll
                for (int I = 0; I < NB; ++I)
                    U[I] -= contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                        [&](int kt) { return ld_frag<E>(Ws + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                        [&](int kt) { return Sb[kt]; });
            }
            F Ub[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) Ub[I] = EL::cvt(U[I]);
            // o = scale (Q*G) S + A U~
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                f32x4 O = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>(Qs + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return Sb[kt]; });
                O = contract(O, I + 1,
                    [&](int kb) { return ld_frag<E>(Aqk + (16 * I + r16) * PC + 16 * kb + 4 * g4); },
                    [&](int kb) { return Ub[kb]; });
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = 16 * I + 4 * g4 + j;
                    if (row < clen) og[(t0 + row) * sv + (int64_t)h * DV + wcol + r16] = EL::from_f(O[j]);
                }
            }
            // S <- Gc (.) S + (K*Gend)^T U~
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                if constexpr (GATE == 2) S[kt] *= ld4(Gc + 16 * kt + 4 * g4);
                else S[kt] *= Gc[0];
                S[kt] = contract(S[kt], NB,
                    [&](int kb) { return ld_frag<E>(KsT + (16 * kt + r16) * PC + 16 * kb + 4 * g4); },
                    [&](int kb) { return Ub[kb]; });
            }
        }
    }

    if (p.ht && wvalid) {
#pragma unroll
        for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                p.ht[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV + wcol + r16] = S[kt][j];
    }
}

template <int DK, int CH, typename E, int GATE>
static hipError_t launch_chunk(const ChunkParams &p, hipStream_t stream) {
    constexpr int NW = 4;
    const int64_t blocks = (int64_t)p.n_seqs * p.H * p.n_tiles;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL((chunk_fwd_kernel<DK, CH, NW, E, GATE>), dim3((unsigned)blocks), dim3(64 * NW),
                       0, stream, p);
    return hipGetLastError();
}

int chunk_tile_cols() { return 64; }

// dtype x dk x chunk x gate dispatch
hipError_t chunk_fwd(int dtype, int dk, int chunk, int gate_vector, const ChunkParams &p,
                     hipStream_t stream) {
#define VGDR_GATES(DK_, CH_, E_)                                                       \
    return gate_vector ? launch_chunk<DK_, CH_, E_, 2>(p, stream)                      \
                       : launch_chunk<DK_, CH_, E_, 1>(p, stream);
    if (dtype == 1) {
        if (dk == 64) { if (chunk == 32) { VGDR_GATES(64, 32, __bf16) } VGDR_GATES(64, 64, __bf16) }
        if (chunk == 32) { VGDR_GATES(128, 32, __bf16) } VGDR_GATES(128, 64, __bf16)
    }
    if (dtype == 2) {
        if (dk == 64) { if (chunk == 32) { VGDR_GATES(64, 32, _Float16) } VGDR_GATES(64, 64, _Float16) }
        if (chunk == 32) { VGDR_GATES(128, 32, _Float16) } VGDR_GATES(128, 64, _Float16)
    }
    // fp32: the 128-key tile only fits LDS with 32-token chunks
    if (dk == 64) { if (chunk == 32) { VGDR_GATES(64, 32, float) } VGDR_GATES(64, 64, float) }
    VGDR_GATES(128, 32, float)
#undef VGDR_GATES
}

}  // namespace vgdr

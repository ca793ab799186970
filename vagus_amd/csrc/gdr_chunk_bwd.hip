// Backward of the chunked gated delta rule, scalar gate or none, delta rule:
// the gradient the reference's training takes through chunk_scan
// (linear_attention.py:237-309, autograd) or fla's chunk backward (the call
// at :487-491 with grads enabled).
//
// Forward, per chunk of CH tokens, in the unified WY form the forward kernels
// use (gdr_chunk.hip), with the in-chunk cumulative log decay gamma,
// D_ij = exp(gamma_i - gamma_j), GX_i = exp(gamma_i), GO_i = scale GX_i,
// GE_i = exp(gamma_C - gamma_i), Gc = exp(gamma_C):
//     N  = strict_lower(K K^T * D)      M = diag(beta) N      TE = (I + M)^-1 diag(beta)
//     A  = scale lower(Q K^T * D)
//     X  = V - diag(GX) K S             U = TE X
//     O  = diag(GO) Q S + A U           S' = Gc S + K^T diag(GE) U
// Backward, given dO and dS' (the gradient of the chunk's exit state):
//     dU = A^T dO + diag(GE) K dS'      dX = TE^T dU          dV = dX
//     dS = Gc dS' + Q^T diag(GO) dO - K^T diag(GX) dX        (chunk to chunk, in reverse)
//     dA = lower(dO U^T)                dTE = dU X^T
//     T0 = (I + M)^-1 = I - TE N        Z = T0^T dTE          dM = -strict_lower(Z TE^T)
//     dbeta_i = Z_ii + sum_j dM_ij N_ij                       dN = diag(beta) dM
//     W_A = scale dA * D                W_N = dN * D
//     dQ = diag(GO) dO S^T + W_A K
//     dK = -diag(GX) dX S^T + diag(GE) U dS'^T + W_A^T Q + (W_N + W_N^T) K
//     dgamma_i = sum_j (dA*A + dN*N)_ij - sum_j (dA*A + dN*N)_ji
//                + GO_i q_i.(dO S^T)_i - GX_i k_i.(dX S^T)_i - GE_i k_i.(U dS'^T)_i
//     dgamma_C += sum_i GE_i k_i.(U dS'^T)_i + Gc <S, dS'>
//     dg_t = sum_{i >= t} dgamma_i        (gamma is the in-chunk cumulative sum of g)
// T0 = I - TE N follows from T0 (I + diag(beta) N) = I, so no division by beta.
//
// Kernels, launched after chunk_prep_kernel has rebuilt TE, A and the gate
// factors of every chunk (the forward's workspace blocks):
//   chunk_hs_kernel   (sequence, head, dv tile): the forward recurrence again,
//                     storing each chunk's entry state S (fp32) in the workspace;
//   chunk_dhs_kernel  (sequence, head, dv tile): the reverse recurrence for dS,
//                     writing dV = dX, each chunk's exit-state gradient and dS0;
//   chunk_grad_kernel (chunk, head), all chunks in parallel: dQ, dK, dbeta, dg
//                     from the chunk's S, dS', dO, dX.
// Products run on the MFMA units in the C-layout convention of gdr_common.hpp:
// element-type operands (bf16 / fp16 / fp32) with fp32 accumulation, and fp32
// operands for the small CH x CH chain (T0, Z, dM), where cancellation makes
// 16-bit rounding of the operands costly.
#include "gdr_chunk_layout.hpp"
#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

namespace {

// CH rows x DK columns of a token-major matrix (row t at src + t * stride) into
// LDS, row-major at rm (pitch prm) and/or transposed at tr (pitch ptr); rows
// >= clen are zero.  Both pitches keep 16-byte rows aligned.
template <typename E, int CH, int DK, int NT>
__device__ __forceinline__ void stage_rows(E *rm, int prm, E *tr, int ptr, const E *src, int64_t stride, int clen,
                                           int tid) {
    constexpr int VE = 16 / (int)sizeof(E);
    typedef E V __attribute__((ext_vector_type(VE)));
    constexpr int UPR = DK / VE;
    for (int u = tid; u < CH * UPR; u += NT) {
        const int row = u / UPR, c0 = (u % UPR) * VE;
        V x = {};
        if (row < clen) x = *reinterpret_cast<const V *>(src + row * stride + c0);
        if (rm) *reinterpret_cast<V *>(rm + row * prm + c0) = x;
        if (tr) {
#pragma unroll
            for (int e = 0; e < VE; ++e) tr[(c0 + e) * ptr + row] = x[e];
        }
    }
}

// position of element (row, col) of a fragment-order CH x CH block (frag_pos)
template <int NB>
__device__ __forceinline__ int blk_pos(int row, int col) {
    return frag_pos<NB>(row >> 4, col >> 4, 16 * ((col & 15) >> 2) + (row & 15)) + (col & 3);
}

// A fragment-order CH x CH block (TE or A, lower triangle with the diagonal)
// as a plain LDS matrix: dst[row][col] (or dst[col][row] when TRANS), zeros
// above the diagonal.  The block is read in order (coalesced).
template <typename E, typename T, int CH, bool TRANS, int NT>
__device__ __forceinline__ void unpack_block(T *dst, int pitch, const E *blk, int tid) {
    constexpr int NB = CH / 16;
    for (int p = tid; p < CH * CH; p += NT) {
        const int e8 = p & 7, ln = (p >> 3) & 63, pr = p >> 9;   // pr = I (NB / 2) + q
        const int I = pr / (NB / 2), q = pr % (NB / 2);
        const int row = 16 * I + (ln & 15), col = 16 * (2 * q + (e8 >> 2)) + 4 * (ln >> 4) + (e8 & 3);
        const float x = col <= row ? (float)blk[p] : 0.f;
        if (TRANS) dst[col * pitch + row] = (T)x;
        else dst[row * pitch + col] = (T)x;
    }
}

// four consecutive rows k0 .. k0 + 3 of column c of a row-major fp32 matrix
__device__ __forceinline__ f32x4 col4(const float *m, int pitch, int k0, int c) {
    return f32x4{m[k0 * pitch + c], m[(k0 + 1) * pitch + c], m[(k0 + 2) * pitch + c], m[(k0 + 3) * pitch + c]};
}

__device__ __forceinline__ float sum16(float x) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) x += __shfl_xor(x, o);
    return x;
}
__device__ __forceinline__ float sum64(float x) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) x += __shfl_xor(x, o);
    return x;
}

// (sequence, head, dv tile) of a walk workgroup; the dv tiles of one
// (sequence, head) share an XCD (the forward state kernel's order)
struct WalkUnit {
    int seq, h, tile;
    int64_t bos, eos, cbase;
};
__device__ __forceinline__ bool walk_unit(const ChunkBwdParams &p, WalkUnit &u) {
    const int b = blockIdx.x;
    const int xcd = b & 7, y = b >> 3;
    const int tile = y % p.n_tiles;
    const int pos = (y / p.n_tiles) * 8 + xcd;
    if (pos >= p.geo.n_seqs * p.H) return false;
    u.h = pos % p.H;
    const int spos = pos / p.H;
    u.seq = p.geo.order ? p.geo.order[spos] : spos;
    seq_bounds(p.geo, u.seq, u.bos, u.eos);
    u.cbase = chunk_base(p.geo, u.seq);
    u.tile = tile;
    return true;
}

// (sequence, chunk within it) of chunk slot `slot` (chunk_prep_kernel's order)
__device__ __forceinline__ bool locate_chunk(const SeqGeom &g, int64_t slot, int &seq, int64_t &cin) {
    if (g.cu) {
        const int32_t *offs = g.chunk_offs;
        if (slot >= offs[g.n_seqs]) return false;
        int lo = 0, hi = g.n_seqs - 1;                          // largest s with offs[s] <= slot
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (offs[mid] <= slot) lo = mid; else hi = mid - 1;
        }
        seq = lo;
        cin = slot - offs[lo];
        return true;
    }
    seq = (int)(slot / g.chunks_per_seq);
    cin = slot % g.chunks_per_seq;
    return seq < g.n_seqs;
}

}  // namespace

// ===========================================================================
// chunk_hs_kernel: entry state of every chunk
// ===========================================================================
template <int DK, int CH, int NW, typename E>
__global__ void __launch_bounds__(64 * NW) chunk_hs_kernel(const ChunkBwdParams p) {
    using EL = Elem<E>;
    using F = typename EL::frag;
    using CB = ChunkBlock<E, CH, DK, 1>;
    constexpr int NT = 64 * NW, NB = CH / 16, NKB = DK / 16, VE = 16 / (int)sizeof(E);
    constexpr int PK = DK + VE, PT = CH + VE;
    __shared__ __attribute__((aligned(16))) E Ks[CH * PK];
    __shared__ __attribute__((aligned(16))) E KT[DK * PT];
    __shared__ __attribute__((aligned(16))) float gx[CH];
    __shared__ __attribute__((aligned(16))) float ge[CH];
    __shared__ float gcs[4];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    WalkUnit u;
    if (!walk_unit(p, u)) return;
    const int H = p.H, DV = p.DV, h = u.h;
    const int col = u.tile * 16 * NW + 16 * wave + r16;
    const bool wvalid = u.tile * 16 * NW + 16 * wave < DV;     // DV % 16 == 0
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * DV;
    const E *kg = reinterpret_cast<const E *>(p.k) + (int64_t)h * DK;
    const E *vg = reinterpret_cast<const E *>(p.v) + (int64_t)h * DV + col;

    f32x4 S[NKB];
    const int64_t sbase = ((int64_t)u.seq * H + h) * DK * DV + col;
#pragma unroll
    for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            S[kt][j] = (p.h0 && wvalid) ? p.h0[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] : 0.f;

    const int nchunks = (int)((u.eos - u.bos + CH - 1) / CH);
    for (int c = 0; c < nchunks; ++c) {
        const int64_t slot = u.cbase + c;
        if (wvalid) {
            float *hs = p.hs + (slot * H + h) * DK * DV + col;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) hs[(int64_t)(16 * kt + 4 * g4 + j) * DV] = S[kt][j];
        }
        if (c + 1 == nchunks) break;                           // the last exit state is not needed
        const int64_t t0 = u.bos + (int64_t)c * CH;
        const int clen = (int)(u.eos - t0 < CH ? u.eos - t0 : CH);
        const char *blkb = reinterpret_cast<const char *>(p.blocks) + (slot * H + h) * CB::BYTES;
        const E *TEb = reinterpret_cast<const E *>(blkb);
        const float *gf = reinterpret_cast<const float *>(blkb + CB::GOFF);
        __syncthreads();                                       // the previous chunk's LDS reads are done
        stage_rows<E, CH, DK, NT>(Ks, PK, KT, PT, kg + t0 * sqk, sqk, clen, tid);
        if (tid < CH) {
            gx[tid] = gf[tid];
            ge[tid] = gf[2 * CH + tid];
        }
        if (tid == 0) gcs[0] = gf[3 * CH];
        __syncthreads();
        if (wvalid) {
            F Sb[NKB];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) Sb[kt] = EL::cvt(S[kt]);
            F Xb[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                const f32x4 P = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>(Ks + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return Sb[kt]; });
                f32x4 X;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = 16 * I + 4 * g4 + j;
                    const float v = row < clen ? EL::to_f(vg[(t0 + row) * sv]) : 0.f;
                    X[j] = v - gx[row] * P[j];
                }
                Xb[I] = EL::cvt(X);
            }
            F Wb[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                const f32x4 U = contract(f32x4{0.f, 0.f, 0.f, 0.f}, I + 1,
                    [&](int kb) { return gfrag<E>(TEb + frag_pos<NB>(I, kb, lane)); },
                    [&](int kb) { return Xb[kb]; });
                Wb[I] = EL::cvt(U * ld4(ge + 16 * I + 4 * g4));
            }
            const float gc = gcs[0];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
                S[kt] = contract(S[kt] * gc, NB,
                    [&](int kb) { return ld_frag<E>(KT + (16 * kt + r16) * PT + 16 * kb + 4 * g4); },
                    [&](int kb) { return Wb[kb]; });
        }
    }
}

// ===========================================================================
// chunk_dhs_kernel: the reverse recurrence for dS; dV = dX
// ===========================================================================
template <int DK, int CH, int NW, typename E>
__global__ void __launch_bounds__(64 * NW) chunk_dhs_kernel(const ChunkBwdParams p) {
    using EL = Elem<E>;
    using F = typename EL::frag;
    using CB = ChunkBlock<E, CH, DK, 1>;
    constexpr int NT = 64 * NW, NB = CH / 16, NKB = DK / 16, VE = 16 / (int)sizeof(E);
    constexpr int PK = DK + VE, PT = CH + VE;
    __shared__ __attribute__((aligned(16))) E Ks[CH * PK];
    __shared__ __attribute__((aligned(16))) E KT[DK * PT];
    __shared__ __attribute__((aligned(16))) E QT[DK * PT];
    __shared__ __attribute__((aligned(16))) E TEt[CH * PT];   // TE^T
    __shared__ __attribute__((aligned(16))) E At[CH * PT];    // A^T
    __shared__ __attribute__((aligned(16))) float gx[CH];
    __shared__ __attribute__((aligned(16))) float go[CH];
    __shared__ __attribute__((aligned(16))) float ge[CH];
    __shared__ float gcs[4];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    WalkUnit u;
    if (!walk_unit(p, u)) return;
    const int H = p.H, DV = p.DV, h = u.h;
    const int col = u.tile * 16 * NW + 16 * wave + r16;
    const bool wvalid = u.tile * 16 * NW + 16 * wave < DV;
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * DV;
    const E *kg = reinterpret_cast<const E *>(p.k) + (int64_t)h * DK;
    const E *qg = reinterpret_cast<const E *>(p.q) + (int64_t)h * DK;
    const E *dog = reinterpret_cast<const E *>(p.dout) + (int64_t)h * DV + col;
    E *dvg = reinterpret_cast<E *>(p.dv) + (int64_t)h * DV + col;

    f32x4 dS[NKB];
    const int64_t sbase = ((int64_t)u.seq * H + h) * DK * DV + col;
#pragma unroll
    for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            dS[kt][j] = (p.dht && wvalid) ? p.dht[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] : 0.f;

    const int nchunks = (int)((u.eos - u.bos + CH - 1) / CH);
    for (int c = nchunks - 1; c >= 0; --c) {
        const int64_t slot = u.cbase + c;
        if (wvalid) {
            float *dhs = p.dhs + (slot * H + h) * DK * DV + col;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) dhs[(int64_t)(16 * kt + 4 * g4 + j) * DV] = dS[kt][j];
        }
        const int64_t t0 = u.bos + (int64_t)c * CH;
        const int clen = (int)(u.eos - t0 < CH ? u.eos - t0 : CH);
        const char *blkb = reinterpret_cast<const char *>(p.blocks) + (slot * H + h) * CB::BYTES;
        const E *TEb = reinterpret_cast<const E *>(blkb);
        const float *gf = reinterpret_cast<const float *>(blkb + CB::GOFF);
        __syncthreads();
        stage_rows<E, CH, DK, NT>(Ks, PK, KT, PT, kg + t0 * sqk, sqk, clen, tid);
        stage_rows<E, CH, DK, NT>(nullptr, 0, QT, PT, qg + t0 * sqk, sqk, clen, tid);
        unpack_block<E, E, CH, true, NT>(TEt, PT, TEb, tid);
        unpack_block<E, E, CH, true, NT>(At, PT, TEb + CH * CH, tid);
        if (tid < CH) {
            gx[tid] = gf[tid];
            go[tid] = gf[CH + tid];
            ge[tid] = gf[2 * CH + tid];
        }
        if (tid == 0) gcs[0] = gf[3 * CH];
        __syncthreads();
        if (wvalid) {
            f32x4 dO[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = 16 * I + 4 * g4 + j;
                    dO[I][j] = row < clen ? EL::to_f(dog[(t0 + row) * sv]) : 0.f;
                }
            F dOb[NB], dSb[NKB];
#pragma unroll
            for (int I = 0; I < NB; ++I) dOb[I] = EL::cvt(dO[I]);
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) dSb[kt] = EL::cvt(dS[kt]);
            // dU = A^T dO + diag(GE) K dS'
            F Yb[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                f32x4 Y = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>(Ks + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return dSb[kt]; });
                Y *= ld4(ge + 16 * I + 4 * g4);
                Y = contract(Y, NB, [&](int kb) { return ld_frag<E>(At + (16 * I + r16) * PT + 16 * kb + 4 * g4); },
                             [&](int kb) { return dOb[kb]; });
                Yb[I] = EL::cvt(Y);
            }
            // dX = TE^T dU  -> dV;  operands of the state update
            F Ob[NB], Xb[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                const f32x4 dX = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NB,
                    [&](int kb) { return ld_frag<E>(TEt + (16 * I + r16) * PT + 16 * kb + 4 * g4); },
                    [&](int kb) { return Yb[kb]; });
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = 16 * I + 4 * g4 + j;
                    if (row < clen) dvg[(t0 + row) * sv] = EL::from_f(dX[j]);
                }
                Ob[I] = EL::cvt(dO[I] * ld4(go + 16 * I + 4 * g4));
                Xb[I] = EL::cvt(-dX * ld4(gx + 16 * I + 4 * g4));
            }
            // dS = Gc dS' + Q^T diag(GO) dO - K^T diag(GX) dX
            const float gc = gcs[0];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                f32x4 s = contract(dS[kt] * gc, NB,
                    [&](int kb) { return ld_frag<E>(QT + (16 * kt + r16) * PT + 16 * kb + 4 * g4); },
                    [&](int kb) { return Ob[kb]; });
                dS[kt] = contract(s, NB,
                    [&](int kb) { return ld_frag<E>(KT + (16 * kt + r16) * PT + 16 * kb + 4 * g4); },
                    [&](int kb) { return Xb[kb]; });
            }
        }
    }
    if (p.dh0 && wvalid) {
#pragma unroll
        for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
            for (int j = 0; j < 4; ++j) p.dh0[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] = dS[kt][j];
    }
}

// ===========================================================================
// chunk_grad_kernel: dQ, dK, dbeta, dg of one (chunk, head)
// ===========================================================================
template <int DK, int CH, typename E>
struct GradLayout {
    static constexpr int ES = sizeof(E), VE = 16 / ES;
    static constexpr int NCW = ES == 2 ? 4 : 2;               // waves of the column phase
    static constexpr int DVB = 16 * NCW;                      // dv columns per block
    static constexpr int PK = DK + VE, PT = CH + VE, PD = DVB + VE, PF = CH + 4;
    // K rows, K^T and Q^T for the whole kernel
    static constexpr int PERS = (CH * PK + 2 * DK * PT) * ES;
    // column phase: A^T; X, U, dU, dO, dX rows of the block; S, dS' rows of the block
    static constexpr int COLS = (CH * PT + 5 * CH * PD + 2 * DK * PD) * ES;
    // CH x CH phase: four fp32 matrices; W_A, W_A^T, W_N + W_N^T in the element type
    static constexpr int SQ = 4 * CH * PF * 4 + 3 * CH * PT * ES;
    static constexpr int REGION = cmax(COLS, SQ);
    static constexpr int SMALL = 8 * CH * 4 + 64;
    static constexpr int BYTES = PERS + REGION + SMALL;
    static_assert(PERS % 16 == 0 && REGION % 16 == 0, "16-byte aligned LDS carving");
    static constexpr bool FITS = BYTES <= 160 * 1024;
};

template <int DK, int CH, typename E>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
chunk_grad_kernel(const ChunkBwdParams p) {
    using L = GradLayout<DK, CH, E>;
    static_assert(L::FITS, "LDS budget exceeded");
    using EL = Elem<E>;
    using F = typename EL::frag;
    using CB = ChunkBlock<E, CH, DK, 1>;
    constexpr int NT = 256, NW = 4, NB = CH / 16, NKB = DK / 16;
    constexpr int NCW = L::NCW, DVB = L::DVB, NKD = DVB / 16;
    constexpr int PK = L::PK, PT = L::PT, PD = L::PD, PF = L::PF;
    constexpr int NL = NB * (NB + 1) / 2, LPW = (NL + NW - 1) / NW;   // lower CH x CH tiles, per wave
    static_assert(NW % NB == 0, "a row block is split over whole waves");
    constexpr int JPW = NB * NKB / NW;                                 // CH x DK tiles per wave

    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    E *Ks = reinterpret_cast<E *>(smem);
    E *KT = Ks + CH * PK;
    E *QT = KT + DK * PT;
    char *R = smem + L::PERS;
    // column phase
    E *At = reinterpret_cast<E *>(R);
    E *Xs = At + CH * PT;
    E *Us = Xs + CH * PD;
    E *Ys = Us + CH * PD;
    E *dOs = Ys + CH * PD;
    E *dXs = dOs + CH * PD;
    E *Ss = dXs + CH * PD;
    E *dSs = Ss + DK * PD;
    // CH x CH phase
    float *Fte = reinterpret_cast<float *>(R);
    float *Fn = Fte + CH * PF;
    float *Fdte = Fn + CH * PF;
    float *Ft0 = Fdte + CH * PF;                  // T0, then Z
    E *WA = reinterpret_cast<E *>(Ft0 + CH * PF);
    E *WAt = WA + CH * PT;
    E *WS = WAt + CH * PT;
    float *sm = reinterpret_cast<float *>(R + L::REGION);
    float *gam = sm, *bet = sm + CH, *gx = sm + 2 * CH, *go = sm + 3 * CH, *ge = sm + 4 * CH;
    float *dgam = sm + 5 * CH, *dbet = sm + 6 * CH;
    float *misc = sm + 8 * CH;                    // [0] Gc, [1] dgamma_C

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    const int H = p.H, DV = p.DV;
    const int h = blockIdx.x % H;
    const int64_t slot = blockIdx.x / H;
    int seq;
    int64_t cin;
    if (!locate_chunk(p.geo, slot, seq, cin)) return;
    int64_t bos, eos;
    seq_bounds(p.geo, seq, bos, eos);
    const int64_t t0 = bos + cin * CH;
    const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * DV;
    const char *blkb = reinterpret_cast<const char *>(p.blocks) + (slot * H + h) * CB::BYTES;
    const E *TEb = reinterpret_cast<const E *>(blkb);
    const E *Ab = TEb + CH * CH;
    const float *gf = reinterpret_cast<const float *>(blkb + CB::GOFF);
    const float *hsb = p.hs + (slot * H + h) * DK * DV;
    const float *dhsb = p.dhs + (slot * H + h) * DK * DV;

    // ---- stage ------------------------------------------------------------
    stage_rows<E, CH, DK, NT>(Ks, PK, KT, PT, reinterpret_cast<const E *>(p.k) + t0 * sqk + (int64_t)h * DK, sqk,
                              clen, tid);
    stage_rows<E, CH, DK, NT>(nullptr, 0, QT, PT, reinterpret_cast<const E *>(p.q) + t0 * sqk + (int64_t)h * DK,
                              sqk, clen, tid);
    unpack_block<E, E, CH, true, NT>(At, PT, Ab, tid);
    if (tid < CH) {
        gx[tid] = gf[tid];
        go[tid] = gf[CH + tid];
        ge[tid] = gf[2 * CH + tid];
        bet[tid] = tid < clen ? p.beta[(t0 + tid) * H + h] : 0.f;
        dgam[tid] = 0.f;
        dbet[tid] = 0.f;
    }
    if (tid == 0) {
        misc[0] = gf[3 * CH];
        misc[1] = 0.f;
    }
    if (wave == 0) {                                           // gamma: in-chunk inclusive sum of g
        float x = (p.g && lane < clen) ? p.g[(t0 + lane) * H + h] : 0.f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        if (lane < CH) gam[lane] = x;
    }
    __syncthreads();

    // ---- column phase: dv blocks of DVB columns ---------------------------
    // wave w < NCW computes X, U, dU (and loads S, dS', dO, dX) for columns
    // 16 w .. 16 w + 15 of the block; then every wave accumulates its tiles of
    // the products that contract over dv.
    const int Iw = wave % NB, J0 = (wave / NB) * JPW;          // this wave's C x DK tiles (Iw, J0 + s)
    f32x4 aQ[JPW], aX[JPW], aE[JPW];                           // dO S^T, dX S^T, U dS'^T
    f32x4 aA[LPW], aT[LPW];                                    // dO U^T, dU X^T (lower tiles)
#pragma unroll
    for (int s = 0; s < JPW; ++s) aQ[s] = aX[s] = aE[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < LPW; ++s) aA[s] = aT[s] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto tile_of = [&](int l, int &I, int &J) __attribute__((always_inline)) {
        I = 0;
        J = l;
        while (J > I) { J -= I + 1; ++I; }
    };
    float gcacc = 0.f;
    const int ndb = (DV + DVB - 1) / DVB;
    for (int db = 0; db < ndb; ++db) {
        const int cb = db * DVB;
        if (db > 0) __syncthreads();                           // the previous block's reads are done
        if (wave < NCW) {
            const int cw = 16 * wave + r16;                      // column within the block
            const int col = cb + cw;
            const bool cv = cb + 16 * wave < DV;
            f32x4 S[NKB], dSx[NKB];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t off = (int64_t)(16 * kt + 4 * g4 + j) * DV + col;
                    S[kt][j] = cv ? hsb[off] : 0.f;
                    dSx[kt][j] = cv ? dhsb[off] : 0.f;
                }
            F Sb[NKB], dSb[NKB];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                gcacc += S[kt][0] * dSx[kt][0] + S[kt][1] * dSx[kt][1] + S[kt][2] * dSx[kt][2] +
                         S[kt][3] * dSx[kt][3];
                Sb[kt] = EL::cvt(S[kt]);
                dSb[kt] = EL::cvt(dSx[kt]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    Ss[(16 * kt + 4 * g4 + j) * PD + cw] = EL::from_f(S[kt][j]);
                    dSs[(16 * kt + 4 * g4 + j) * PD + cw] = EL::from_f(dSx[kt][j]);
                }
            }
            F Xb[NB], dOb[NB];
            f32x4 X[NB], Y[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                const f32x4 P = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>(Ks + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return Sb[kt]; });
                const f32x4 P2 = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>(Ks + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return dSb[kt]; });
                f32x4 dO;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = 16 * I + 4 * g4 + j;
                    const bool ok = cv && row < clen;
                    const int64_t off = (t0 + row) * sv + (int64_t)h * DV + col;
                    const float v = ok ? EL::to_f(reinterpret_cast<const E *>(p.v)[off]) : 0.f;
                    dO[j] = ok ? EL::to_f(reinterpret_cast<const E *>(p.dout)[off]) : 0.f;
                    const float dx = ok ? EL::to_f(reinterpret_cast<const E *>(p.dv)[off]) : 0.f;
                    X[I][j] = v - gx[row] * P[j];
                    Y[I][j] = ge[row] * P2[j];
                    Xs[row * PD + cw] = EL::from_f(X[I][j]);
                    dOs[row * PD + cw] = EL::from_f(dO[j]);
                    dXs[row * PD + cw] = EL::from_f(dx);
                }
                Xb[I] = EL::cvt(X[I]);
                dOb[I] = EL::cvt(dO);
            }
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                // U = TE X ;  dU = A^T dO + diag(GE) K dS'
                const f32x4 U = contract(f32x4{0.f, 0.f, 0.f, 0.f}, I + 1,
                    [&](int kb) { return gfrag<E>(TEb + frag_pos<NB>(I, kb, lane)); },
                    [&](int kb) { return Xb[kb]; });
                Y[I] = contract(Y[I], NB,
                    [&](int kb) { return ld_frag<E>(At + (16 * I + r16) * PT + 16 * kb + 4 * g4); },
                    [&](int kb) { return dOb[kb]; });
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = 16 * I + 4 * g4 + j;
                    Us[row * PD + cw] = EL::from_f(U[j]);
                    Ys[row * PD + cw] = EL::from_f(Y[I][j]);
                }
            }
        }
        __syncthreads();
        // products contracting over the block's columns
#pragma unroll
        for (int s = 0; s < JPW; ++s) {
            const int J = J0 + s;
            aQ[s] = contract(aQ[s], NKD,
                [&](int kb) { return ld_frag<E>(dOs + (16 * Iw + r16) * PD + 16 * kb + 4 * g4); },
                [&](int kb) { return ld_frag<E>(Ss + (16 * J + r16) * PD + 16 * kb + 4 * g4); });
            aX[s] = contract(aX[s], NKD,
                [&](int kb) { return ld_frag<E>(dXs + (16 * Iw + r16) * PD + 16 * kb + 4 * g4); },
                [&](int kb) { return ld_frag<E>(Ss + (16 * J + r16) * PD + 16 * kb + 4 * g4); });
            aE[s] = contract(aE[s], NKD,
                [&](int kb) { return ld_frag<E>(Us + (16 * Iw + r16) * PD + 16 * kb + 4 * g4); },
                [&](int kb) { return ld_frag<E>(dSs + (16 * J + r16) * PD + 16 * kb + 4 * g4); });
        }
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            const int l = wave + NW * s;
            if (l < NL) {
                int I, J;
                tile_of(l, I, J);
                aA[s] = contract(aA[s], NKD,
                    [&](int kb) { return ld_frag<E>(dOs + (16 * I + r16) * PD + 16 * kb + 4 * g4); },
                    [&](int kb) { return ld_frag<E>(Us + (16 * J + r16) * PD + 16 * kb + 4 * g4); });
                aT[s] = contract(aT[s], NKD,
                    [&](int kb) { return ld_frag<E>(Ys + (16 * I + r16) * PD + 16 * kb + 4 * g4); },
                    [&](int kb) { return ld_frag<E>(Xs + (16 * J + r16) * PD + 16 * kb + 4 * g4); });
            }
        }
    }
    __syncthreads();                                           // the region now holds the CH x CH phase

    // ---- CH x CH phase ----------------------------------------------------
    for (int i = tid; i < 3 * CH * PF; i += NT) Fn[i] = 0.f;   // N, dTE, T0 (written by lower tiles)
    for (int i = tid; i < 3 * CH * PT; i += NT) WA[i] = EL::from_f(0.f);
    unpack_block<E, float, CH, false, NT>(Fte, PF, TEb, tid);
    {
        const float t = sum64(gcacc);
        if (lane == 0 && wave < NCW) atomicAdd(&misc[1], misc[0] * t);     // Gc <S, dS'>
    }
    __syncthreads();
    // dA: the A terms of dgamma; W_A = scale dA * D kept in aA.  dTE -> Fdte.  N -> Fn.
#pragma unroll
    for (int s = 0; s < LPW; ++s) {
        const int l = wave + NW * s;
        if (l < NL) {
            int I, J;
            tile_of(l, I, J);
            const int jj = 16 * J + r16;
            const f32x4 kk = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                [&](int kt) { return ld_frag<E>(Ks + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                [&](int kt) { return ld_frag<E>(Ks + (16 * J + r16) * PK + 16 * kt + 4 * g4); });
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * I + 4 * g4 + j;
                const bool low = jj <= i;
                const float D = low ? __expf(gam[i] - gam[jj]) : 0.f;
                const float da = low ? aA[s][j] : 0.f;
                const float v = low ? da * EL::to_f(Ab[blk_pos<NB>(i, jj)]) : 0.f;
                if (low) {
                    atomicAdd(&dgam[i], v);
                    atomicAdd(&dgam[jj], -v);
                }
                aA[s][j] = p.scale * da * D;
                Fdte[i * PF + jj] = low ? aT[s][j] : 0.f;
                Fn[i * PF + jj] = jj < i ? kk[j] * D : 0.f;
            }
        }
    }
    __syncthreads();
    // T0 = I - TE N (lower tiles)
#pragma unroll
    for (int s = 0; s < LPW; ++s) {
        const int l = wave + NW * s;
        if (l < NL) {
            int I, J;
            tile_of(l, I, J);
            f32x4 t = {0.f, 0.f, 0.f, 0.f};
            for (int kb = J; kb <= I; ++kb)
                t = mfma_kb1(ld4(Fte + (16 * I + r16) * PF + 16 * kb + 4 * g4),
                             col4(Fn, PF, 16 * kb + 4 * g4, 16 * J + r16), t);
            const int jj = 16 * J + r16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * I + 4 * g4 + j;
                Ft0[i * PF + jj] = jj <= i ? (i == jj ? 1.f : 0.f) - t[j] : 0.f;
            }
        }
    }
    __syncthreads();
    // Z = T0^T dTE (lower tiles); dbeta_i += Z_ii
    f32x4 zt[LPW];
#pragma unroll
    for (int s = 0; s < LPW; ++s) {
        zt[s] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int l = wave + NW * s;
        if (l < NL) {
            int I, J;
            tile_of(l, I, J);
            for (int kb = I; kb < NB; ++kb)
                zt[s] = mfma_kb1(col4(Ft0, PF, 16 * kb + 4 * g4, 16 * I + r16),
                                 col4(Fdte, PF, 16 * kb + 4 * g4, 16 * J + r16), zt[s]);
            if (I == J) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (4 * g4 + j == r16) atomicAdd(&dbet[16 * I + r16], zt[s][j]);
            }
        }
    }
    __syncthreads();                                           // T0 and dTE are consumed
    float *Fz = Ft0;
#pragma unroll
    for (int s = 0; s < LPW; ++s) {
        const int l = wave + NW * s;
        if (l < NL) {
            int I, J;
            tile_of(l, I, J);
#pragma unroll
            for (int j = 0; j < 4; ++j) Fz[(16 * I + 4 * g4 + j) * PF + 16 * J + r16] = zt[s][j];
        }
    }
    __syncthreads();
    // dM = -strict_lower(Z TE^T): the M terms of dbeta and dgamma, W_N + W_N^T -> WS; W_A -> WA, WA^T
#pragma unroll
    for (int s = 0; s < LPW; ++s) {
        const int l = wave + NW * s;
        if (l < NL) {
            int I, J;
            tile_of(l, I, J);
            f32x4 m = {0.f, 0.f, 0.f, 0.f};
            for (int kb = 0; kb <= J; ++kb)
                m = mfma_kb1(ld4(Fz + (16 * I + r16) * PF + 16 * kb + 4 * g4),
                             ld4(Fte + (16 * J + r16) * PF + 16 * kb + 4 * g4), m);
            const int jj = 16 * J + r16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * I + 4 * g4 + j;
                if (jj < i) {
                    const float dm = -m[j];
                    const float n = Fn[i * PF + jj];
                    atomicAdd(&dbet[i], dm * n);
                    const float dn = bet[i] * dm;
                    atomicAdd(&dgam[i], dn * n);
                    atomicAdd(&dgam[jj], -dn * n);
                    const E wn = EL::from_f(dn * __expf(gam[i] - gam[jj]));
                    WS[i * PT + jj] = wn;
                    WS[jj * PT + i] = wn;
                }
                if (jj <= i) {
                    const E wa = EL::from_f(aA[s][j]);
                    WA[i * PT + jj] = wa;
                    WAt[jj * PT + i] = wa;
                }
            }
        }
    }
    __syncthreads();

    // ---- dQ, dK of this wave's tiles, and their dgamma terms --------------
    {
        float rq[4] = {0.f, 0.f, 0.f, 0.f}, rx[4] = {0.f, 0.f, 0.f, 0.f}, re[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < JPW; ++s) {
            const int d = 16 * (J0 + s) + r16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * Iw + 4 * g4 + j;
                const float qv = EL::to_f(QT[d * PT + i]), kv = EL::to_f(Ks[i * PK + d]);
                rq[j] += qv * aQ[s][j];
                rx[j] += kv * aX[s][j];
                re[j] += kv * aE[s][j];
            }
        }
        float ce = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = 16 * Iw + 4 * g4 + j;
            const float q1 = sum16(rq[j]), x1 = sum16(rx[j]), e1 = sum16(re[j]);
            if (r16 == 0) atomicAdd(&dgam[i], go[i] * q1 - gx[i] * x1 - ge[i] * e1);
            ce += ge[i] * e1;
        }
        if (r16 == 0) atomicAdd(&misc[1], ce);
    }
    E *dqg = reinterpret_cast<E *>(p.dq) + t0 * sqk + (int64_t)h * DK;
    E *dkg = reinterpret_cast<E *>(p.dk) + t0 * sqk + (int64_t)h * DK;
    const f32x4 GOr = ld4(go + 16 * Iw + 4 * g4), GXr = ld4(gx + 16 * Iw + 4 * g4), GEr = ld4(ge + 16 * Iw + 4 * g4);
#pragma unroll
    for (int s = 0; s < JPW; ++s) {
        const int J = J0 + s;
        f32x4 q = contract(aQ[s] * GOr, NB,
            [&](int kb) { return ld_frag<E>(WA + (16 * Iw + r16) * PT + 16 * kb + 4 * g4); },
            [&](int kb) { return ld_frag<E>(KT + (16 * J + r16) * PT + 16 * kb + 4 * g4); });
        f32x4 k = contract(aE[s] * GEr - aX[s] * GXr, NB,
            [&](int kb) { return ld_frag<E>(WAt + (16 * Iw + r16) * PT + 16 * kb + 4 * g4); },
            [&](int kb) { return ld_frag<E>(QT + (16 * J + r16) * PT + 16 * kb + 4 * g4); });
        k = contract(k, NB,
            [&](int kb) { return ld_frag<E>(WS + (16 * Iw + r16) * PT + 16 * kb + 4 * g4); },
            [&](int kb) { return ld_frag<E>(KT + (16 * J + r16) * PT + 16 * kb + 4 * g4); });
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = 16 * Iw + 4 * g4 + j;
            if (i < clen) {
                dqg[i * sqk + 16 * J + r16] = EL::from_f(q[j]);
                dkg[i * sqk + 16 * J + r16] = EL::from_f(k[j]);
            }
        }
    }
    __syncthreads();
    // ---- dg (suffix sums of dgamma; gamma_C is gamma at the last token) and dbeta
    if (wave == 0) {
        float x = lane < clen ? dgam[lane] : 0.f;
        if (lane == clen - 1) x += misc[1];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_down(x, o);
            if (lane + o < 64) x += y;
        }
        if (lane < clen) {
            if (p.dg) p.dg[(t0 + lane) * H + h] = x;
            p.dbeta[(t0 + lane) * H + h] = dbet[lane];
        }
    }
}

// ===========================================================================
// launch
// ===========================================================================
template <int DK, int CH, typename E>
static hipError_t run_bwd(ChunkBwdParams p, hipStream_t stream) {
    const int64_t units = (int64_t)p.geo.n_seqs * p.H;
    const int nw = units * ((p.DV + 63) / 64) >= device_cu_count() ? 4 : 2;
    p.n_tiles = (p.DV + 16 * nw - 1) / (16 * nw);
    const int64_t walk_blocks = (units + 7) / 8 * 8 * p.n_tiles;
    if (walk_blocks > 0) {
        if (nw == 4) {
            hipLaunchKernelGGL((chunk_hs_kernel<DK, CH, 4, E>), dim3((unsigned)walk_blocks), dim3(256), 0, stream, p);
            hipLaunchKernelGGL((chunk_dhs_kernel<DK, CH, 4, E>), dim3((unsigned)walk_blocks), dim3(256), 0, stream, p);
        } else {
            hipLaunchKernelGGL((chunk_hs_kernel<DK, CH, 2, E>), dim3((unsigned)walk_blocks), dim3(128), 0, stream, p);
            hipLaunchKernelGGL((chunk_dhs_kernel<DK, CH, 2, E>), dim3((unsigned)walk_blocks), dim3(128), 0, stream, p);
        }
    }
    const int64_t grad_blocks = (int64_t)p.n_chunk_slots * p.H;
    if (grad_blocks > 0)
        hipLaunchKernelGGL((chunk_grad_kernel<DK, CH, E>), dim3((unsigned)grad_blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t chunk_bwd(int dtype, int dk, int chunk, const ChunkParams &fwd, ChunkBwdParams p, int32_t *table,
                     hipStream_t stream) {
    if (p.geo.n_seqs == 0) return hipSuccess;
    // TE, A and the gate factors of every chunk, as the forward built them
    hipError_t e = chunk_fwd(dtype, dk, chunk, 0, fwd, table, CHUNK_PREP, stream);
    if (e != hipSuccess) return e;
    if (p.geo.cu) {
        p.geo.chunk_offs = table + 2 * p.geo.n_seqs;
        p.geo.order = table + 3 * p.geo.n_seqs + 1;
    }
#define VGDR_BWD(DK_, CH_, E_) return run_bwd<DK_, CH_, E_>(p, stream);
    if (dtype == 1) {
        if (dk == 64) { if (chunk == 32) { VGDR_BWD(64, 32, __bf16) } VGDR_BWD(64, 64, __bf16) }
        if (chunk == 32) { VGDR_BWD(128, 32, __bf16) } VGDR_BWD(128, 64, __bf16)
    }
    if (dtype == 2) {
        if (dk == 64) { if (chunk == 32) { VGDR_BWD(64, 32, _Float16) } VGDR_BWD(64, 64, _Float16) }
        if (chunk == 32) { VGDR_BWD(128, 32, _Float16) } VGDR_BWD(128, 64, _Float16)
    }
    if (dk == 64) { VGDR_BWD(64, 32, float) }
    VGDR_BWD(128, 32, float)
#undef VGDR_BWD
}

}  // namespace vgdr

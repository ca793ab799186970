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
//                     storing each chunk's entry state S in the workspace;
//   chunk_dhs_kernel  (sequence, head, dv tile): the reverse recurrence for dS,
//                     writing dV = dX, each chunk's exit-state gradient and dS0;
//   chunk_grad_kernel (chunk, head), all chunks in parallel: dQ, dK, dbeta, dg
//                     from the chunk's S, dS', dO, dX.
// The workspace states are stored in the element type, in the C-layout
// fragment order of ckpt_pos: the gradient kernel rounds them to that type for
// its products anyway, and a wavefront's 16 columns are one contiguous store
// per key block.  The
// two walks run compute waves beside producer waves that stage each chunk's
// operands into a double-buffered LDS slot.
// Products run on the MFMA units in the C-layout convention of gdr_common.hpp:
// element-type operands (bf16 / fp16 / fp32) with fp32 accumulation, and fp32
// operands for the small CH x CH chain (T0, Z, dM), where cancellation makes
// 16-bit rounding of the operands costly.
#include "gdr_chunk_layout.hpp"
#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

namespace {

// Rows [0, CH) x columns [0, DK) of a row-major matrix (row t at src + t *
// stride), held in registers between load() and store().  load() issues every
// 16-byte load at once, unconditionally, from clamped addresses (a load under
// a per-lane branch waits for the ones before it); store() writes the rows to
// LDS (pitch keeps 16-byte rows aligned) with rows >= `rows` and columns >=
// `cols` zeroed.
template <typename E, int CH, int DK, int NT>
struct RowRegs {
    static constexpr int VE = 16 / (int)sizeof(E), UPR = DK / VE, UNITS = CH * UPR, N = (UNITS + NT - 1) / NT;
    typedef E V __attribute__((ext_vector_type(VE)));
    V x[N];
    __device__ __forceinline__ void load(const E *src, int64_t stride, int rows, int tid, int cols = DK) {
        unroll<N>([&](auto i) __attribute__((always_inline)) {
            const int u = tid + (int)i * NT;
            const int row = u / UPR, c0 = (u % UPR) * VE;
            const bool ok = u < UNITS && row < rows && c0 < cols;
            x[i] = *reinterpret_cast<const V *>(src + (ok ? row * stride + c0 : 0));
        });
    }
    __device__ __forceinline__ void store(E *dst, int pitch, int rows, int tid, int cols = DK) const {
        unroll<N>([&](auto i) __attribute__((always_inline)) {
            const int u = tid + (int)i * NT;
            if (u < UNITS) {
                const int row = u / UPR, c0 = (u % UPR) * VE;
                *reinterpret_cast<V *>(dst + row * pitch + c0) = (row < rows && c0 < cols) ? x[i] : V{};
            }
        });
    }
    // rows in the paired-column order of chunk prep's gated tiles (16-byte unit
    // pu = 4 q + g holds columns 32 q + 4 g .. + 3 and 32 q + 16 + 4 g .. + 3),
    // written to LDS in natural column order
    __device__ __forceinline__ void store_unpaired(E *dst, int pitch, int tid) const {
        static_assert(VE == 8 && DK % 32 == 0, "paired rows are 16-bit, 32-column groups");
        typedef E V4 __attribute__((ext_vector_type(4)));
        unroll<N>([&](auto i) __attribute__((always_inline)) {
            const int u = tid + (int)i * NT;
            if (u < UNITS) {
                const int row = u / UPR, pu = u % UPR, c0 = 32 * (pu >> 2) + 4 * (pu & 3);
                *reinterpret_cast<V4 *>(dst + row * pitch + c0) = __builtin_shufflevector(x[i], x[i], 0, 1, 2, 3);
                *reinterpret_cast<V4 *>(dst + row * pitch + c0 + 16) = __builtin_shufflevector(x[i], x[i], 4, 5, 6, 7);
            }
        });
    }
};

// NCB column blocks (16 columns each) of a state checkpoint (ckpt_pos order, a
// contiguous run) in registers; store() writes them as an LDS matrix
// dst[c][d] (column c of the blocks, key row d; pitch keeps 8-byte fragments
// aligned), column blocks >= `ncb` zeroed.
template <typename E, int DK, int NCB, int NT>
struct CkptRegs {
    static constexpr int VE = 16 / (int)sizeof(E), UNITS = NCB * DK * 16 / VE, N = (UNITS + NT - 1) / NT;
    static constexpr int NKB = DK / 16;
    typedef E V __attribute__((ext_vector_type(VE)));
    V x[N];
    __device__ __forceinline__ void load(const E *src, int ncb, int tid) {
        unroll<N>([&](auto i) __attribute__((always_inline)) {
            const int u = tid + (int)i * NT;
            const bool ok = u < UNITS && u * VE / (DK * 16) < ncb;
            x[i] = *reinterpret_cast<const V *>(src + (ok ? u * VE : 0));
        });
    }
    __device__ __forceinline__ void store(E *dst, int pitch, int ncb, int tid) const {
        using F = typename Elem<E>::frag;
        unroll<N>([&](auto i) __attribute__((always_inline)) {
            const int u = tid + (int)i * NT;
            if (u < UNITS) {
#pragma unroll
                for (int hh = 0; hh < VE / 4; ++hh) {
                    const int e0 = u * VE + 4 * hh;               // ckpt_pos(cb, kt, l) of these four
                    const int l = (e0 >> 2) & 63, kt = (e0 >> 8) % NKB, cb = e0 / (256 * NKB);
                    F f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) f[e] = cb < ncb ? x[i][4 * hh + e] : E(0.f);
                    *reinterpret_cast<F *>(dst + (16 * cb + (l & 15)) * pitch + 16 * kt + 4 * (l >> 4)) = f;
                }
            }
        });
    }
};

// A fragment-order CH x CH block (TE or A: lower triangle with the diagonal)
// in registers, 16-byte units read in order; store() writes it as a plain
// row-major LDS matrix.  A fragment is four consecutive columns of one row,
// so each is one 8-byte (16-bit types) or 16-byte (fp32) store.  Tiles above
// the diagonal are written as zeros (chunk_prep leaves them unwritten, except
// the partner of a diagonal tile pair, and zeros inside the diagonal tiles).
//
// LIVE (16-bit, four row blocks): only the six tile pairs (I, q) with 2 q <= I
// are copied (unit n of the copy is unit n % 64 of the (n / 64)-th of them);
// the other two pairs hold only tiles above the diagonal, zero_dead() writes
// their tiles as zeros once and no later store touches them.
template <typename E, int CH, int NT, bool LIVE = false>
struct BlockRegs {
    static constexpr int VE = 16 / (int)sizeof(E), ALL = CH * CH / VE;
    static constexpr int NB = CH / 16;
    static_assert(!LIVE || (sizeof(E) == 2 && NB == 4), "live pairs: 16-bit, 64-token blocks");
    static constexpr int UNITS = LIVE ? 384 : ALL, N = (UNITS + NT - 1) / NT;
    typedef E V __attribute__((ext_vector_type(VE)));
    V x[N];
    // unit of the block that copy unit n holds
    __device__ static __forceinline__ int unit(int n) {
        if constexpr (LIVE) {
            const int j = n >> 6;                                          // 0..5 -> pairs 0, 2, 4, 5, 6, 7
            return ((j == 0 ? 0 : (j == 1 ? 2 : j + 2)) << 6) + (n & 63);
        } else {
            return n;
        }
    }
    __device__ __forceinline__ void load(const E *blk, int tid) {
        unroll<N>([&](auto i) __attribute__((always_inline)) {
            const int n = tid + (int)i * NT;
            x[i] = *reinterpret_cast<const V *>(blk + unit(n < UNITS ? n : 0) * VE);
        });
    }
    // the tiles of the pairs LIVE skips: rows 0 .. 31, columns 32 .. 63
    __device__ static __forceinline__ void zero_dead(E *dst, int pitch, int tid) {
        if constexpr (LIVE) {
            using F = typename Elem<E>::frag;
            for (int f = tid; f < 32 * 8; f += NT) {                       // 4-column fragments
                const int row = f >> 3, c = 32 + 4 * (f & 7);
                *reinterpret_cast<F *>(dst + row * pitch + c) = F{};
            }
        }
    }
    __device__ __forceinline__ void store(E *dst, int pitch, int tid) const {
        using F = typename Elem<E>::frag;
        unroll<N>([&](auto i) __attribute__((always_inline)) {
            const int n = tid + (int)i * NT, u = unit(n);
            if (n < UNITS) {
                const int p = u * VE;                              // first element of the unit
                const int ln = (p >> 3) & 63, pr = p >> 9;         // pr = I (NB / 2) + q
                const int I = pr / (NB / 2), q = pr % (NB / 2);
                const int row = 16 * I + (ln & 15);
#pragma unroll
                for (int h = 0; h < VE / 4; ++h) {                 // the unit's fragments (two for 16-bit types)
                    const int kb = 2 * q + ((p >> 2) & 1) + h;
                    F f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) f[e] = kb <= I ? x[i][4 * h + e] : E(0.f);
                    *reinterpret_cast<F *>(dst + row * pitch + 16 * kb + 4 * (ln >> 4)) = f;
                }
            }
        });
    }
};

// four consecutive elements to global memory (aligned to their size)
template <typename E>
__device__ __forceinline__ void st_gfrag(E *p, typename Elem<E>::frag x) {
    *reinterpret_cast<typename Elem<E>::frag *>(p) = x;
}

// position of element (row, col) of a fragment-order CH x CH block (frag_pos)
template <int NB>
__device__ __forceinline__ int blk_pos(int row, int col) {
    return frag_pos<NB>(row >> 4, col >> 4, 16 * ((col & 15) >> 2) + (row & 15)) + (col & 3);
}

// LDS row pitch (elements) of an N-column matrix: 288-byte rows for N = 128 in
// a 16-bit type, at which both the 8-byte fragment reads of 16 rows and the
// transpose reads run conflict-free on gfx950
template <typename E, int N>
struct Pitch {
    static constexpr int value = N + (sizeof(E) == 2 ? 16 : 4);
};

// Lane (g, r) gets M[k0 + 4 g + j][c0 + r], j = 0..3, of a row-major LDS
// matrix M (pitch pm): the A-operand fragment of M^T at row c0 + r, or the
// B-operand fragment of M at column c0 + r, over the k-block of rows k0 ..
// k0 + 15.  16-bit types use the transpose read; fp32 reads four rows.
template <typename E>
__device__ __forceinline__ typename Elem<E>::frag ld_colfrag(const E *M, int pm, int k0, int c0, int lane) {
    const int g = lane >> 4, s = lane & 15;
    if constexpr (sizeof(E) == 2) {
        return ld_tr<E>(M + (k0 + 4 * g + (s >> 2)) * pm + c0 + 4 * (s & 3));
    } else {
        const E *b = M + (k0 + 4 * g) * pm + c0 + s;
        return typename Elem<E>::frag{b[0], b[pm], b[2 * pm], b[3 * pm]};
    }
}

// four consecutive rows k0 .. k0 + 3 of column c of a row-major fp32 matrix
__device__ __forceinline__ f32x4 col4(const float *m, int pitch, int k0, int c) {
    return f32x4{m[k0 * pitch + c], m[(k0 + 1) * pitch + c], m[(k0 + 2) * pitch + c], m[(k0 + 3) * pitch + c]};
}

// the sum over the 16 lanes of x's row, in every lane of the row (DPP)
__device__ __forceinline__ float sum16(float x) { return row_sum16(x); }
// the sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (one lane of each row)
__device__ __forceinline__ float sum_rows(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ float sum64(float x) { return sum_rows(sum16(x)); }

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
template <int V_> struct SlotTag { static constexpr int value = V_; };

// NWC compute waves (16 state columns each) re-run the forward recurrence and
// store each chunk's entry state; NWC producer waves stage each chunk's K rows,
// the tile's V rows and the gate factors into the idle half of a
// double-buffered LDS slot (one barrier per chunk hands a slot over; separate
// loops, equal barrier counts).  The compute waves load their own TE fragments
// one chunk ahead.  (They had loaded V too, two bytes per load in the MFMA
// layout.)
template <int DK, int CH, int NWC, typename E>
__global__ void __launch_bounds__(128 * NWC) chunk_hs_kernel(const ChunkBwdParams p) {
    using EL = Elem<E>;
    using F = typename EL::frag;
    using CB = ChunkBlock<E, CH, DK, 1>;
    constexpr int NTP = 64 * NWC, NB = CH / 16, NKB = DK / 16;
    constexpr int PK = Pitch<E, DK>::value;
    constexpr int DW = 16 * NWC, PD = DW + 8;                  // the tile's V columns, their LDS pitch
    __shared__ __attribute__((aligned(16))) E Ks0[CH * PK];
    __shared__ __attribute__((aligned(16))) E Ks1[CH * PK];
    __shared__ __attribute__((aligned(16))) float gt0[3 * CH + 4];   // GX, GO, GE, then Gc
    __shared__ __attribute__((aligned(16))) float gt1[3 * CH + 4];
    __shared__ __attribute__((aligned(16))) E Vs0[CH * PD];
    __shared__ __attribute__((aligned(16))) E Vs1[CH * PD];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    WalkUnit u;
    if (!walk_unit(p, u)) return;
    const int H = p.H, DV = p.DV, h = u.h;
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * DV;
    const int nchunks = (int)((u.eos - u.bos + CH - 1) / CH);
    const int nsteps = nchunks > 0 ? nchunks - 1 : 0;          // the last chunk's exit state is not needed
    auto clen_of = [&](int c) __attribute__((always_inline)) {
        const int64_t t0 = u.bos + (int64_t)c * CH;
        return (int)(u.eos - t0 < CH ? u.eos - t0 : CH);
    };
    auto blk_of = [&](int c) __attribute__((always_inline)) {
        return reinterpret_cast<const char *>(p.blocks) + ((u.cbase + c) * H + h) * CB::BYTES;
    };

    if (wave >= NWC) {
        // ---- producers ----------------------------------------------------
        const int ptid = tid - 64 * NWC;
        const E *kg = reinterpret_cast<const E *>(p.k) + (int64_t)h * DK;
        constexpr int NG = 3 * CH + 1, GPT = (NG + NTP - 1) / NTP;   // gate floats, per producer thread
        RowRegs<E, CH, DK, NTP> rk;
        RowRegs<E, CH, DW, NTP> rv;
        const int cb = u.tile * DW;
        const E *vt = reinterpret_cast<const E *>(p.v) + (int64_t)h * DV + cb;
        float gv[GPT];
        auto fetch = [&](int c) __attribute__((always_inline)) {
            rk.load(kg + (u.bos + (int64_t)c * CH) * sqk, sqk, clen_of(c), ptid);
            rv.load(vt + (u.bos + (int64_t)c * CH) * sv, sv, clen_of(c), ptid, DV - cb);
#pragma unroll
            for (int i = 0; i < GPT; ++i) {
                const int gi = ptid + i * NTP;
                gv[i] = reinterpret_cast<const float *>(blk_of(c) + CB::GOFF)[gi < NG ? gi : 0];
            }
        };
        auto put = [&](auto tag, int c) __attribute__((always_inline)) {
            constexpr int SL = decltype(tag)::value;
            rk.store(SL ? Ks1 : Ks0, PK, clen_of(c), ptid);
            rv.store(SL ? Vs1 : Vs0, PD, clen_of(c), ptid, DV - cb);   // zero past the chunk's end and dv
#pragma unroll
            for (int i = 0; i < GPT; ++i)
                if (ptid + i * NTP < NG) (SL ? gt1 : gt0)[ptid + i * NTP] = gv[i];
        };
        if (nsteps == 0) return;
        fetch(0);
        put(SlotTag<0>{}, 0);
        __syncthreads();
        for (int k = 0; k < nsteps; k += 2) {
            if (k + 1 < nsteps) {                              // step k reads slot 0: fill slot 1
                fetch(k + 1);
                put(SlotTag<1>{}, k + 1);
            }
            __syncthreads();
            if (k + 1 < nsteps) {
                if (k + 2 < nsteps) {                          // step k + 1 reads slot 1: fill slot 0
                    fetch(k + 2);
                    put(SlotTag<0>{}, k + 2);
                }
                __syncthreads();
            }
        }
        return;
    }

    // ---- compute waves ------------------------------------------------------
    const int colw = u.tile * 16 * NWC + 16 * wave;
    const bool wvalid = colw < DV;                             // DV % 16 == 0
    const int col = wvalid ? colw + r16 : r16;                 // in bounds for the unconditional loads
    f32x4 S[NKB];
    const int64_t sbase = ((int64_t)u.seq * H + h) * DK * DV + col;
#pragma unroll
    for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            S[kt][j] = (p.h0 && wvalid) ? p.h0[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] : 0.f;
    auto store_state = [&](int c) __attribute__((always_inline)) {
        if constexpr (sizeof(E) == 2) {
            // branch-free (a wave past dv stores into a zero-byte resource), so the
            // next wait for this wave's loads does not wait for these stores too
            const __amdgpu_buffer_rsrc_t rs =
                buffer_rsrc(reinterpret_cast<E *>(p.hs) + ((u.cbase + c) * H + h) * (int64_t)DK * DV,
                            wvalid ? (uint32_t)(DK * DV * sizeof(E)) : 0u);
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
                buffer_store_8b(EL::cvt(S[kt]), rs, (uint32_t)(ckpt_pos<DK>(colw >> 4, kt, lane) * sizeof(E)));
        } else if (wvalid) {
            E *hs = reinterpret_cast<E *>(p.hs) + ((u.cbase + c) * H + h) * (int64_t)DK * DV;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) st_gfrag<E>(hs + ckpt_pos<DK>(colw >> 4, kt, lane), EL::cvt(S[kt]));
        }
    };
    // TE fragments (lower tiles) of the next chunk, raw: a conversion next to
    // its load would wait for every load before it
    F ten[NB * NB];
    auto fetch_own = [&](int c) __attribute__((always_inline)) {
        const E *TEb = reinterpret_cast<const E *>(blk_of(c));
#pragma unroll
        for (int I = 0; I < NB; ++I)
#pragma unroll
            for (int kb = 0; kb <= I; ++kb) ten[I * NB + kb] = gfrag<E>(TEb + frag_pos<NB>(I, kb, lane));
    };
    auto step = [&](auto tag, int c) __attribute__((always_inline)) {
        constexpr int SL = decltype(tag)::value;
        const E *Ks = SL ? Ks1 : Ks0;
        const float *gt = SL ? gt1 : gt0;
        store_state(c);
        // V rows 16 I + 4 g .. + 3 of column r (the B-operand layout; zero past the end)
        const E *Vs = SL ? Vs1 : Vs0;
        f32x4 V[NB];
        F TEf[NB * NB];
#pragma unroll
        for (int I = 0; I < NB; ++I) {
            V[I] = EL::tof(ld_colfrag<E>(Vs, PD, 16 * I, 16 * wave, lane));
#pragma unroll
            for (int kb = 0; kb <= I; ++kb) TEf[I * NB + kb] = ten[I * NB + kb];
        }
        if (c + 1 < nsteps) fetch_own(c + 1);
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
                Xb[I] = EL::cvt(V[I] - ld4(gt + 16 * I + 4 * g4) * P);
            }
            F Wb[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                const f32x4 U = contract(f32x4{0.f, 0.f, 0.f, 0.f}, I + 1,
                    [&](int kb) { return TEf[I * NB + kb]; },
                    [&](int kb) { return Xb[kb]; });
                Wb[I] = EL::cvt(U * ld4(gt + 2 * CH + 16 * I + 4 * g4));
            }
            const float gc = gt[3 * CH];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
                S[kt] = contract(S[kt] * gc, NB,
                    [&](int kb) { return ld_colfrag<E>(Ks, PK, 16 * kb, 16 * kt, lane); },
                    [&](int kb) { return Wb[kb]; });
        }
    };
    if (nsteps > 0) {
        fetch_own(0);
        __syncthreads();                                       // slot 0 holds chunk 0
    }
    for (int k = 0; k < nsteps; k += 2) {
        step(SlotTag<0>{}, k);
        __syncthreads();
        if (k + 1 < nsteps) {
            step(SlotTag<1>{}, k + 1);
            __syncthreads();
        }
    }
    if (nchunks > 0) store_state(nchunks - 1);
}

// ===========================================================================
// chunk_dhs_kernel: the reverse recurrence for dS; dV = dX
// ===========================================================================

// NWC compute waves (16 state columns each) and NWC producer waves.  The
// producers load each chunk's K, Q rows, TE and A blocks, gate factors and the
// tile's dO rows into registers and stage them into the idle half of a
// double-buffered LDS slot while the compute waves work on the other half; one
// barrier per chunk hands a slot over.  The two roles run separate loops with
// the same barrier count.  (The compute waves had loaded dO themselves, two
// bytes per load in the MFMA layout: 22 us more at gdn_340m.)  16-bit dV
// leaves as 16-byte units: the compute waves also form dX^T = dU^T TE (the dX
// product with its operands swapped), whose C layout gives a lane four
// consecutive columns of one token, and pair token blocks through
// v_permlane16_swap for eight.
// VEC (per-channel gate, 16-bit): the operands are chunk prep's gated tiles
// instead of K and Q rows with per-row factors: K*G (Ks) and scale Q*G (Qs)
// for dS, K*Gend (KEs) for dU, and Gc per key channel:
//     dU = A^T dO + (K*Gend) dS'     dS = diag(Gc) dS' + (scale Q*G)^T dO - (K*G)^T dX
template <int DK, int CH, int NWC, typename E, bool VEC = false, int NPW = NWC>
__global__ void __launch_bounds__(64 * (NWC + NPW)) chunk_dhs_kernel(const ChunkBwdParams p) {
    using EL = Elem<E>;
    using F = typename EL::frag;
    using CB = ChunkBlock<E, CH, DK, VEC ? 2 : 1>;
    static_assert(!VEC || CB::VEC, "the per-channel walk reads the 16-bit gated tiles");
    constexpr int NTP = 64 * NPW, NB = CH / 16, NKB = DK / 16;
    constexpr int PK = Pitch<E, DK>::value, PT = Pitch<E, CH>::value;
    constexpr int NGF = VEC ? DK : 3 * CH + 4;
    constexpr int DW = 16 * NWC, PD = DW + 8;                  // the tile's dO columns, their LDS pitch
    __shared__ __attribute__((aligned(16))) E Ks0[CH * PK];
    __shared__ __attribute__((aligned(16))) E Ks1[CH * PK];
    __shared__ __attribute__((aligned(16))) E Qs0[CH * PK];
    __shared__ __attribute__((aligned(16))) E Qs1[CH * PK];
    __shared__ __attribute__((aligned(16))) E KE0[VEC ? CH * PK : 8];
    __shared__ __attribute__((aligned(16))) E KE1[VEC ? CH * PK : 8];
    __shared__ __attribute__((aligned(16))) E TE0[CH * PT];
    __shared__ __attribute__((aligned(16))) E TE1[CH * PT];
    __shared__ __attribute__((aligned(16))) E Am0[CH * PT];
    __shared__ __attribute__((aligned(16))) E Am1[CH * PT];
    __shared__ __attribute__((aligned(16))) float gt0[NGF];          // GX, GO, GE, then Gc (VEC: Gc per channel)
    __shared__ __attribute__((aligned(16))) float gt1[NGF];
    __shared__ __attribute__((aligned(16))) E dO0[CH * PD];
    __shared__ __attribute__((aligned(16))) E dO1[CH * PD];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    WalkUnit u;
    if (!walk_unit(p, u)) return;
    const int H = p.H, DV = p.DV, h = u.h;
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * DV;
    const int nchunks = (int)((u.eos - u.bos + CH - 1) / CH);
    auto clen_of = [&](int c) __attribute__((always_inline)) {
        const int64_t t0 = u.bos + (int64_t)c * CH;
        return (int)(u.eos - t0 < CH ? u.eos - t0 : CH);
    };

    if (wave >= NWC) {
        // ---- producers ----------------------------------------------------
        const int ptid = tid - 64 * NWC;
        const E *kg = reinterpret_cast<const E *>(p.k) + (int64_t)h * DK;
        const E *qg = reinterpret_cast<const E *>(p.q) + (int64_t)h * DK;
        const int cb = u.tile * DW;
        const E *dot = reinterpret_cast<const E *>(p.dout) + (int64_t)h * DV + cb;
        constexpr bool LIVEB = sizeof(E) == 2 && CH == 64;     // TE, A: the six pairs that can be nonzero
        using BR = BlockRegs<E, CH, NTP, LIVEB>;
        constexpr int NG = VEC ? DK : 3 * CH + 1, GPT = (NG + NTP - 1) / NTP;   // gate floats, per producer thread
        // one chunk's operands in registers; two sets, so that each chunk's loads
        // are issued two steps before its LDS slot is filled (with one set, each
        // fill waited for loads issued just before it)
        struct Stage {
            RowRegs<E, CH, DK, NTP> rk, rq;
            RowRegs<E, CH, VEC ? DK : 32, NTP> rke;             // VEC: K*Gend rows
            RowRegs<E, CH, DW, NTP> rdo;                        // dO rows, the tile's columns
            BR rte, ra;
            float gv[GPT];
        };
        auto fetch = [&](Stage &st, int c) __attribute__((always_inline)) {
            const int64_t t0 = u.bos + (int64_t)c * CH;
            const int clen = clen_of(c);
            const char *blkb = reinterpret_cast<const char *>(p.blocks) + ((u.cbase + c) * H + h) * CB::BYTES;
            if constexpr (VEC) {
                const E *tiles = reinterpret_cast<const E *>(blkb) + CB::TEA;      // K*G, scale Q*G, K*Gend
                st.rk.load(tiles, DK, CH, ptid);
                st.rq.load(tiles + CH * DK, DK, CH, ptid);
                st.rke.load(tiles + 2 * CH * DK, DK, CH, ptid);
            } else {
                st.rk.load(kg + t0 * sqk, sqk, clen, ptid);
                st.rq.load(qg + t0 * sqk, sqk, clen, ptid);
            }
            st.rte.load(reinterpret_cast<const E *>(blkb), ptid);
            st.ra.load(reinterpret_cast<const E *>(blkb) + CH * CH, ptid);
            st.rdo.load(dot + t0 * sv, sv, clen, ptid, DV - cb);
#pragma unroll
            for (int i = 0; i < GPT; ++i) {
                const int gi = ptid + i * NTP;
                st.gv[i] = reinterpret_cast<const float *>(blkb + CB::GOFF)[gi < NG ? gi : 0];
            }
        };
        auto put = [&](auto tag, const Stage &st, int c) __attribute__((always_inline)) {
            constexpr int SL = decltype(tag)::value;
            const int clen = clen_of(c);
            if constexpr (VEC) {
                st.rk.store_unpaired(SL ? Ks1 : Ks0, PK, ptid);
                st.rq.store(SL ? Qs1 : Qs0, PK, CH, ptid);
                st.rke.store_unpaired(SL ? KE1 : KE0, PK, ptid);
            } else {
                st.rk.store(SL ? Ks1 : Ks0, PK, clen, ptid);
                st.rq.store(SL ? Qs1 : Qs0, PK, clen, ptid);
            }
            st.rte.store(SL ? TE1 : TE0, PT, ptid);
            st.ra.store(SL ? Am1 : Am0, PT, ptid);
            st.rdo.store(SL ? dO1 : dO0, PD, clen, ptid, DV - cb);   // zero past the chunk's end and dv
#pragma unroll
            for (int i = 0; i < GPT; ++i)
                if (ptid + i * NTP < NG) (SL ? gt1 : gt0)[ptid + i * NTP] = st.gv[i];
        };
        if (nchunks == 0) return;
        BR::zero_dead(TE0, PT, ptid);
        BR::zero_dead(TE1, PT, ptid);
        BR::zero_dead(Am0, PT, ptid);
        BR::zero_dead(Am1, PT, ptid);
        // step k works on chunk n - 1 - k from slot k & 1, filled during step k - 1
        // from register set k & 1, whose loads were issued during step k - 2
        auto chunk_of = [&](int k) __attribute__((always_inline)) { return nchunks - 1 - k; };
        Stage s0, s1;
        fetch(s0, chunk_of(0));
        if (1 < nchunks) fetch(s1, chunk_of(1));
        put(SlotTag<0>{}, s0, chunk_of(0));
        __syncthreads();
        for (int k = 0; k < nchunks; k += 2) {
            if (k + 2 < nchunks) fetch(s0, chunk_of(k + 2));
            if (k + 1 < nchunks) put(SlotTag<1>{}, s1, chunk_of(k + 1));
            __syncthreads();                                   // end of step k
            if (k + 1 < nchunks) {
                if (k + 3 < nchunks) fetch(s1, chunk_of(k + 3));
                if (k + 2 < nchunks) put(SlotTag<0>{}, s0, chunk_of(k + 2));
                __syncthreads();                               // end of step k + 1
            }
        }
        return;
    }

    // ---- compute waves ------------------------------------------------------
    const int colw = u.tile * 16 * NWC + 16 * wave;
    const bool wvalid = colw < DV;
    const int col = wvalid ? colw + r16 : r16;
    E *dvg = reinterpret_cast<E *>(p.dv) + (int64_t)h * DV + col;
    f32x4 dS[NKB];
    const int64_t sbase = ((int64_t)u.seq * H + h) * DK * DV + col;
#pragma unroll
    for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            dS[kt][j] = (p.dht && wvalid) ? p.dht[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] : 0.f;
    auto step = [&](auto tag, int k) __attribute__((always_inline)) {
        constexpr int SL = decltype(tag)::value;
        const E *Ks = SL ? Ks1 : Ks0;
        const E *Qs = SL ? Qs1 : Qs0;
        const E *KEs = VEC ? (SL ? KE1 : KE0) : Ks;
        const E *TEm = SL ? TE1 : TE0;
        const E *Am = SL ? Am1 : Am0;
        const float *gt = SL ? gt1 : gt0;
        const int c = nchunks - 1 - k;
        const int64_t slot = u.cbase + c;
        const int64_t t0 = u.bos + (int64_t)c * CH;
        const int clen = clen_of(c);
        if constexpr (sizeof(E) == 2) {
            // branch-free (a wave past dv stores into a zero-byte resource): a store
            // under a branch made the join below wait for it to reach memory
            const __amdgpu_buffer_rsrc_t rs =
                buffer_rsrc(reinterpret_cast<E *>(p.dhs) + (slot * H + h) * (int64_t)DK * DV,
                            wvalid ? (uint32_t)(DK * DV * sizeof(E)) : 0u);
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
                buffer_store_8b(EL::cvt(dS[kt]), rs, (uint32_t)(ckpt_pos<DK>(colw >> 4, kt, lane) * sizeof(E)));
        } else if (wvalid) {
            E *dhs = reinterpret_cast<E *>(p.dhs) + (slot * H + h) * (int64_t)DK * DV;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) st_gfrag<E>(dhs + ckpt_pos<DK>(colw >> 4, kt, lane), EL::cvt(dS[kt]));
        }
        if (wvalid) {
            // dO rows 16 I + 4 g .. + 3 of column r (the B-operand layout; zero past the end)
            const E *dOs = SL ? dO1 : dO0;
            f32x4 dO[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) dO[I] = EL::tof(ld_colfrag<E>(dOs, PD, 16 * I, 16 * wave, lane));
            F dOb[NB], dSb[NKB];
#pragma unroll
            for (int I = 0; I < NB; ++I) dOb[I] = EL::cvt(dO[I]);
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) dSb[kt] = EL::cvt(dS[kt]);
            // dU = A^T dO + diag(GE) K dS'   (VEC: (K*Gend) dS')
            F Yb[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                f32x4 Y = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>(KEs + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return dSb[kt]; });
                if constexpr (!VEC) Y *= ld4(gt + 2 * CH + 16 * I + 4 * g4);
                Y = contract(Y, NB, [&](int kb) { return ld_colfrag<E>(Am, PT, 16 * kb, 16 * I, lane); },
                             [&](int kb) { return dOb[kb]; });
                Yb[I] = EL::cvt(Y);
            }
            // dX = TE^T dU  -> dV;  operands of the state update
            F Ob[NB], Xb[NB];
            if constexpr (sizeof(E) == 2) {
                // dV: dX^T = dU^T TE, lane (g, r) holding columns 4 g .. + 3 of token
                // 16 I + r; token blocks 2 m and 2 m + 1 trade halves (lanes l and
                // l ^ 16), after which a lane holds columns 8 (g >> 1) .. + 7 of token
                // 16 (2 m + (g & 1)) + r.  Rows past the chunk's end fall outside the
                // resource (no branch).
                static_assert(NB % 2 == 0, "token blocks go in pairs");
                const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(
                    reinterpret_cast<E *>(p.dv) + t0 * sv + (int64_t)h * DV, (uint32_t)(clen * sv * sizeof(E)));
#pragma unroll
                for (int m = 0; m < NB / 2; ++m) {
                    u32x2 xt[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int I = 2 * m + e;
                        const f32x4 dXT = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NB, [&](int kb) { return Yb[kb]; },
                            [&](int kb) { return ld_colfrag<E>(TEm, PT, 16 * kb, 16 * I, lane); });
                        xt[e] = __builtin_bit_cast(u32x2, EL::cvt(dXT));
                    }
                    const auto a = __builtin_amdgcn_permlane16_swap(xt[0][0], xt[1][0], false, false);
                    const auto b = __builtin_amdgcn_permlane16_swap(xt[0][1], xt[1][1], false, false);
                    const int tok = 16 * (2 * m + (g4 & 1)) + r16, cc = colw + 8 * (g4 >> 1);
                    __builtin_amdgcn_raw_buffer_store_b128(u32x4{a[0], b[0], a[1], b[1]}, rv,
                                                           (int)((tok * sv + cc) * sizeof(E)), 0, 0);
                }
            }
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                const f32x4 dX = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NB,
                    [&](int kb) { return ld_colfrag<E>(TEm, PT, 16 * kb, 16 * I, lane); },
                    [&](int kb) { return Yb[kb]; });
                if constexpr (sizeof(E) != 2) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int row = 16 * I + 4 * g4 + j;
                        if (row < clen) dvg[(t0 + row) * sv] = EL::from_f(dX[j]);
                    }
                }
                if constexpr (VEC) {                           // the factors are in the tiles
                    Ob[I] = EL::cvt(dO[I]);
                    Xb[I] = EL::cvt(-dX);
                } else {
                    Ob[I] = EL::cvt(dO[I] * ld4(gt + CH + 16 * I + 4 * g4));
                    Xb[I] = EL::cvt(-dX * ld4(gt + 16 * I + 4 * g4));
                }
            }
            // dS = Gc dS' + Q^T diag(GO) dO - K^T diag(GX) dX   (VEC: Gc per key channel, gated tiles)
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                const f32x4 dsg = VEC ? dS[kt] * ld4(gt + 16 * kt + 4 * g4) : dS[kt] * gt[3 * CH];
                f32x4 s = contract(dsg, NB,
                    [&](int kb) { return ld_colfrag<E>(Qs, PK, 16 * kb, 16 * kt, lane); },
                    [&](int kb) { return Ob[kb]; });
                dS[kt] = contract(s, NB,
                    [&](int kb) { return ld_colfrag<E>(Ks, PK, 16 * kb, 16 * kt, lane); },
                    [&](int kb) { return Xb[kb]; });
            }
        }
    };
    if (nchunks > 0) __syncthreads();                          // slot 0 holds the last chunk
    for (int k = 0; k < nchunks; k += 2) {
        step(SlotTag<0>{}, k);
        __syncthreads();
        if (k + 1 < nchunks) {
            step(SlotTag<1>{}, k + 1);
            __syncthreads();
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
    static constexpr int PK = Pitch<E, DK>::value, PT = Pitch<E, CH>::value, PV = Pitch<E, DVB>::value;
    static constexpr int PF = CH + 4;
    // K and Q rows, and TE rows (lower tiles), for the whole kernel
    static constexpr int PERS = (2 * CH * PK + CH * PT) * ES;
    // column phase: A; the block's V, dO, dX rows (CH tokens, row-major); its
    // columns of X, U, dU (CH tokens each) and of S, dS' (DK key channels
    // each), stored column by column
    static constexpr int COLS = (CH * PT + 3 * CH * PV + 3 * DVB * PT + 2 * DVB * PK) * ES;
    // CH x CH phase: N, dTE, T0 (then Z) in fp32; W_A and W_N + W_N^T in the element type
    static constexpr int SQ = 3 * CH * PF * 4 + 2 * CH * PT * ES;
    static constexpr int REGION = cmax(COLS, SQ);
    static constexpr int SMALL = 8 * CH * 4 + 64;
    static constexpr int BYTES = PERS + REGION + SMALL;
    static_assert(PERS % 16 == 0 && REGION % 16 == 0, "16-byte aligned LDS carving");
    static constexpr bool FITS = BYTES <= 160 * 1024;
};

// Eight waves, two per SIMD: the kernel's phases are chains of short products
// with LDS round trips in between, and a second wave on each SIMD covers them
// (one workgroup per CU: its LDS is above half of the CU's).
//
// VEC (per-channel gate, 16-bit): only the staging and the column phase run,
// with chunk prep's gated tiles K*G in place of K (P = (K*G) S, X = V - P) and
// K*Gend in place of Q's slot (dU = A^T dO + (K*Gend) dS'); the sums over dv
// (dO S^T, dX S^T, U dS'^T, dO U^T, dU X^T, and per key channel the sum of
// S * dS') go to p.gw for chunk_grad_vec_kernel.
template <int DK, int CH, typename E, bool VEC = false>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
chunk_grad_kernel(const ChunkBwdParams p) {
    using L = GradLayout<DK, CH, E>;
    static_assert(L::FITS, "LDS budget exceeded");
    using EL = Elem<E>;
    using F = typename EL::frag;
    using CB = ChunkBlock<E, CH, DK, VEC ? 2 : 1>;
    static_assert(!VEC || CB::VEC, "the per-channel column phase reads the 16-bit gated tiles");
    constexpr int NT = 512, NW = 8, NB = CH / 16, NKB = DK / 16, NBH = NB / 2;
    constexpr int NCW = L::NCW, DVB = L::DVB, NKD = DVB / 16;
    constexpr int PK = L::PK, PT = L::PT, PV = L::PV, PF = L::PF;
    constexpr int NL = NB * (NB + 1) / 2, LPW = (NL + NW - 1) / NW;   // lower CH x CH tiles, per wave
    static_assert(NW % NB == 0, "a row block is split over whole waves");
    constexpr int JPW = NB * NKB / NW;                                 // CH x DK tiles per wave

    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    E *Ks = reinterpret_cast<E *>(smem);
    E *Qs = Ks + CH * PK;
    E *TEs = Qs + CH * PK;                        // TE rows (zero above the diagonal)
    char *R = smem + L::PERS;
    // column phase
    E *Am = reinterpret_cast<E *>(R);
    E *Vs = Am + CH * PT;                         // V, dO, dX rows of the block
    E *dOs = Vs + CH * PV;
    E *dXs = dOs + CH * PV;
    E *Xs = dXs + CH * PV;                        // Xs[c][t] = X[t][c], c a column of the block
    E *Us = Xs + DVB * PT;
    E *Ys = Us + DVB * PT;
    E *Ss = Ys + DVB * PT;                        // Ss[c][d] = S[d][c]
    E *dSs = Ss + DVB * PK;
    // CH x CH phase
    // N, dTE and T0 are stored transposed (element (i, j) at [j][i]), so that the
    // products below read their column operands as 16-byte rows; Z row-major
    float *Fn = reinterpret_cast<float *>(R);
    float *Fdte = Fn + CH * PF;
    float *Ft0 = Fdte + CH * PF;                  // T0 (transposed), then Z
    E *WA = reinterpret_cast<E *>(Ft0 + CH * PF);
    E *WS = WA + CH * PT;
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
    const E *hsb = reinterpret_cast<const E *>(p.hs) + (slot * H + h) * DK * DV;
    const E *dhsb = reinterpret_cast<const E *>(p.dhs) + (slot * H + h) * DK * DV;

    // ---- stage: every load of the chunk issued at once --------------------
    // (VEC: Ks holds K*G and Qs K*Gend, from the gated tiles)
    RowRegs<E, CH, DK, NT> rk, rq;
    BlockRegs<E, CH, NT> ra, rte;                              // A, TE
    if constexpr (VEC) {
        rk.load(TEb + CB::TEA, DK, CH, tid);
        rq.load(TEb + CB::TEA + 2 * CH * DK, DK, CH, tid);
    } else {
        rk.load(reinterpret_cast<const E *>(p.k) + t0 * sqk + (int64_t)h * DK, sqk, clen, tid);
        rq.load(reinterpret_cast<const E *>(p.q) + t0 * sqk + (int64_t)h * DK, sqk, clen, tid);
    }
    ra.load(Ab, tid);
    rte.load(TEb, tid);
    const int tc = tid < CH ? tid : 0, tg = tc < clen ? tc : 0;
    const float gx_v = VEC ? 0.f : gf[tc], go_v = VEC ? 0.f : gf[CH + tc], ge_v = VEC ? 0.f : gf[2 * CH + tc];
    const float gc_v = VEC ? 0.f : gf[3 * CH];
    const float be_raw = (VEC || !p.beta) ? 0.f : p.beta[(t0 + tg) * H + h];   // no delta rule: beta 0
    const float be_v = p.fz.beta_sigmoid ? sigmoidf_(be_raw) : be_raw;
    const float g_v = (!VEC && p.g) ? p.g[(t0 + (lane < clen ? lane : 0)) * H + h] : 0.f;
    const int Iw = wave % NB, J0 = (wave / NB) * JPW;          // this wave's C x DK tiles (Iw, J0 + s)
    auto tile_of = [&](int l, int &I, int &J) __attribute__((always_inline)) {
        I = 0;
        J = l;
        while (J > I) { J -= I + 1; ++I; }
    };
    // The column phase's global operands of one dv block, as whole 16-byte
    // units: S and dS' columns (the checkpoints' contiguous runs), and the V, dO,
    // dX rows.  Loaded a dv block ahead: block 0 with the staging loads, block
    // db + 1 during block db's products.
    const int cwave = wave & 3, half = wave >> 2;
    const bool colw_ok = cwave < NCW;
    CkptRegs<E, DK, NCW, NT> cS, cdS;
    RowRegs<E, CH, DVB, NT> cV, cdO, cdX;
    auto colload = [&](int db) __attribute__((always_inline)) {
        const int cb = db * DVB, ncol = DV - cb < DVB ? DV - cb : DVB;
        cS.load(hsb + (int64_t)cb * DK, ncol >> 4, tid);        // ckpt_pos(cb / 16, 0, 0) = cb DK
        cdS.load(dhsb + (int64_t)cb * DK, ncol >> 4, tid);
        const int64_t rb = t0 * sv + (int64_t)h * DV + cb;
        cV.load(reinterpret_cast<const E *>(p.v) + rb, sv, clen, tid, ncol);
        cdO.load(reinterpret_cast<const E *>(p.dout) + rb, sv, clen, tid, ncol);
        cdX.load(reinterpret_cast<const E *>(p.dv) + rb, sv, clen, tid, ncol);
    };
    auto colstore = [&](int db) __attribute__((always_inline)) {
        const int cb = db * DVB, ncol = DV - cb < DVB ? DV - cb : DVB;
        cS.store(Ss, PK, ncol >> 4, tid);
        cdS.store(dSs, PK, ncol >> 4, tid);
        cV.store(Vs, PV, clen, tid, ncol);
        cdO.store(dOs, PV, clen, tid, ncol);
        cdX.store(dXs, PV, clen, tid, ncol);
    };
    colload(0);
    if constexpr (VEC) {
        rk.store_unpaired(Ks, PK, tid);
        rq.store_unpaired(Qs, PK, tid);
        if (tid < DK) sm[tid] = 0.f;                           // per-channel sums of S * dS'
    } else {
        rk.store(Ks, PK, clen, tid);
        rq.store(Qs, PK, clen, tid);
    }
    ra.store(Am, PT, tid);
    rte.store(TEs, PT, tid);
    if (!VEC && tid < CH) {
        gx[tid] = gx_v;
        go[tid] = go_v;
        ge[tid] = ge_v;
        bet[tid] = tid < clen ? be_v : 0.f;
        dgam[tid] = 0.f;
        dbet[tid] = 0.f;
    }
    if (!VEC && tid == 0) {
        misc[0] = gc_v;
        misc[1] = 0.f;
    }
    if (!VEC && wave == 0) {                                   // gamma: in-chunk inclusive sum of g
        const float x = wave_scan(lane < clen ? g_v : 0.f);
        if (lane < CH) gam[lane] = x;
    }
    __syncthreads();
    // A at this wave's dA elements (the A terms of dgamma): rows 16 I + 4 g .. + 3
    // of column 16 J + r of the staged A block (zero above the diagonal), one
    // transpose read per tile
    typename EL::frag aval[LPW];
    if constexpr (!VEC) {
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            const int l = wave + NW * s;
            int I = 0, J = 0;
            if (l < NL) tile_of(l, I, J);
            aval[s] = ld_colfrag<E>(Am, PT, 16 * I, 16 * J, lane);
        }
    }

    // ---- column phase: dv blocks of DVB columns ---------------------------
    // then every wave accumulates its tiles of the products that contract over dv
    f32x4 aQ[JPW], aX[JPW], aE[JPW];                           // dO S^T, dX S^T, U dS'^T
    f32x4 aA[LPW], aT[LPW];                                    // dO U^T, dU X^T (lower tiles)
#pragma unroll
    for (int s = 0; s < JPW; ++s) aQ[s] = aX[s] = aE[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < LPW; ++s) aA[s] = aT[s] = f32x4{0.f, 0.f, 0.f, 0.f};
    float gcacc = 0.f;
    float gcv[VEC ? NKB : 1][4] = {};                          // VEC: S * dS' per key channel of this lane
    const int ndb = (DV + DVB - 1) / DVB;
    const int cw = 16 * cwave + r16;                           // column within the block
    for (int db = 0; db < ndb; ++db) {
        if (db > 0) __syncthreads();                           // the previous block's reads are done
        colstore(db);
        __syncthreads();
        f32x4 Y0[NBH];
        if (colw_ok) {
            F Sb[NKB], dSb[NKB];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                Sb[kt] = ld_frag<E>(Ss + cw * PK + 16 * kt + 4 * g4);
                dSb[kt] = ld_frag<E>(dSs + cw * PK + 16 * kt + 4 * g4);
                if (half == 0) {
                    const f32x4 a = EL::tof(Sb[kt]), b = EL::tof(dSb[kt]);
                    if constexpr (VEC) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) gcv[kt][j] += a[j] * b[j];
                    } else {
                        gcacc += a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
                    }
                }
            }
#pragma unroll
            for (int ii = 0; ii < NBH; ++ii) {
                const int I = half * NBH + ii;
                const f32x4 P = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>(Ks + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return Sb[kt]; });
                const f32x4 P2 = contract(f32x4{0.f, 0.f, 0.f, 0.f}, NKB,
                    [&](int kt) { return ld_frag<E>((VEC ? Qs : Ks) + (16 * I + r16) * PK + 16 * kt + 4 * g4); },
                    [&](int kt) { return dSb[kt]; });
                const f32x4 V = EL::tof(ld_colfrag<E>(Vs, PV, 16 * I, 16 * cwave, lane));
                if constexpr (VEC) {
                    st_frag<E>(Xs + cw * PT + 16 * I + 4 * g4, EL::cvt(V - P));
                    Y0[ii] = P2;
                } else {
                    st_frag<E>(Xs + cw * PT + 16 * I + 4 * g4, EL::cvt(V - ld4(gx + 16 * I + 4 * g4) * P));
                    Y0[ii] = ld4(ge + 16 * I + 4 * g4) * P2;
                }
            }
        }
        __syncthreads();                                       // X of both halves in LDS
        if (colw_ok) {
#pragma unroll
            for (int ii = 0; ii < NBH; ++ii) {
                // U = TE X ;  dU = A^T dO + diag(GE) K dS'
                const int I = half * NBH + ii;
                const f32x4 U = contract(f32x4{0.f, 0.f, 0.f, 0.f}, I + 1,
                    [&](int kb) { return ld_frag<E>(TEs + (16 * I + r16) * PT + 16 * kb + 4 * g4); },
                    [&](int kb) { return ld_frag<E>(Xs + cw * PT + 16 * kb + 4 * g4); });
                const f32x4 Y = contract(Y0[ii], NB,
                    [&](int kb) { return ld_colfrag<E>(Am, PT, 16 * kb, 16 * I, lane); },
                    [&](int kb) { return ld_colfrag<E>(dOs, PV, 16 * kb, 16 * cwave, lane); });
                st_frag<E>(Us + cw * PT + 16 * I + 4 * g4, EL::cvt(U));
                st_frag<E>(Ys + cw * PT + 16 * I + 4 * g4, EL::cvt(Y));
            }
        }
        if (db + 1 < ndb) colload(db + 1);
        __syncthreads();
        // products contracting over the block's columns
#pragma unroll
        for (int s = 0; s < JPW; ++s) {
            const int J = J0 + s;
            aQ[s] = contract(aQ[s], NKD,
                             [&](int kb) { return ld_frag<E>(dOs + (16 * Iw + r16) * PV + 16 * kb + 4 * g4); },
                             [&](int kb) { return ld_colfrag<E>(Ss, PK, 16 * kb, 16 * J, lane); });
            aX[s] = contract(aX[s], NKD,
                             [&](int kb) { return ld_frag<E>(dXs + (16 * Iw + r16) * PV + 16 * kb + 4 * g4); },
                             [&](int kb) { return ld_colfrag<E>(Ss, PK, 16 * kb, 16 * J, lane); });
            aE[s] = contract(aE[s], NKD, [&](int kb) { return ld_colfrag<E>(Us, PT, 16 * kb, 16 * Iw, lane); },
                             [&](int kb) { return ld_colfrag<E>(dSs, PK, 16 * kb, 16 * J, lane); });
        }
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            const int l = wave + NW * s;
            if (l < NL) {
                int I, J;
                tile_of(l, I, J);
                aA[s] = contract(aA[s], NKD,
                                 [&](int kb) { return ld_frag<E>(dOs + (16 * I + r16) * PV + 16 * kb + 4 * g4); },
                                 [&](int kb) { return ld_colfrag<E>(Us, PT, 16 * kb, 16 * J, lane); });
                aT[s] = contract(aT[s], NKD, [&](int kb) { return ld_colfrag<E>(Ys, PT, 16 * kb, 16 * I, lane); },
                                 [&](int kb) { return ld_colfrag<E>(Xs, PT, 16 * kb, 16 * J, lane); });
            }
        }
    }
    __syncthreads();                                           // the region now holds the CH x CH phase

    if constexpr (VEC) {
        // the sums over dv for chunk_grad_vec_kernel
        float *gwb = p.gw + (slot * H + h) * grad_vec_work_floats(CH, DK);
        float *gQ = gwb, *gX = gwb + CH * DK, *gE = gwb + 2 * CH * DK;
        float *gA = gwb + 3 * CH * DK, *gT = gA + CH * CH, *gC = gT + CH * CH;
        // dO S^T, dX S^T, U dS'^T transposed ([DK][CH]): a lane's four C-layout rows
        // of one key are one 16-byte unit (and chunk_grad_vec_kernel reads them so)
#pragma unroll
        for (int s = 0; s < JPW; ++s) {
            const int d = 16 * (J0 + s) + r16, i0 = 16 * Iw + 4 * g4;
            *reinterpret_cast<f32x4 *>(gQ + d * CH + i0) = aQ[s];
            *reinterpret_cast<f32x4 *>(gX + d * CH + i0) = aX[s];
            *reinterpret_cast<f32x4 *>(gE + d * CH + i0) = aE[s];
        }
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            const int l = wave + NW * s;
            if (l < NL) {
                int I, J;
                tile_of(l, I, J);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 16 * I + 4 * g4 + j, jj = 16 * J + r16;
                    gA[i * CH + jj] = aA[s][j];
                    gT[i * CH + jj] = aT[s][j];
                }
            }
        }
        if (half == 0 && colw_ok) {
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float t = sum16(gcv[kt][j]);         // over this wave's 16 columns
                    if (r16 == 0) atomicAdd(&sm[16 * kt + 4 * g4 + j], t);
                }
        }
        __syncthreads();
        if (tid < DK) gC[tid] = sm[tid];
        return;
    }

    // ---- CH x CH phase ----------------------------------------------------
    // Every matrix is written tile by tile over the lower tiles (W_A and WS
    // also over their mirror images) before it is read, and reads stay in the
    // tiles written: no zero fill.  Row and column sums go through shuffles
    // first, so each LDS atomic has distinct addresses across its lanes.
    {
        const float t = sum64(gcacc);
        if (lane == 0 && wave < NCW) atomicAdd(&misc[1], misc[0] * t);     // Gc <S, dS'>
    }
    __syncthreads();
    // dA: the A terms of dgamma; W_A = scale dA * D kept in aA.  dTE -> Fdte.  N -> Fn.
    // D and N of the wave's own tile elements stay in registers for the dM step.
    float Dk[LPW][4], Nk[LPW][4];
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
            float rs[4], cs = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * I + 4 * g4 + j;
                const bool low = jj <= i;
                const float D = low ? __expf(gam[i] - gam[jj]) : 0.f;
                const float da = low ? aA[s][j] : 0.f;
                rs[j] = da * EL::to_f(aval[s][j]);
                cs += rs[j];
                aA[s][j] = p.scale * da * D;
                Fdte[jj * PF + i] = low ? aT[s][j] : 0.f;
                Nk[s][j] = jj < i ? kk[j] * D : 0.f;
                Dk[s][j] = D;
                Fn[jj * PF + i] = Nk[s][j];
            }
            cs = sum_rows(cs);
#pragma unroll
            for (int j = 0; j < 4; ++j) rs[j] = sum16(rs[j]);
            if (r16 == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) atomicAdd(&dgam[16 * I + 4 * g4 + j], rs[j]);
            }
            if (g4 == 0) atomicAdd(&dgam[jj], -cs);
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
                t = mfma_kb1(EL::tof(ld_frag<E>(TEs + (16 * I + r16) * PT + 16 * kb + 4 * g4)),
                             ld4(Fn + (16 * J + r16) * PF + 16 * kb + 4 * g4), t);
            const int jj = 16 * J + r16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * I + 4 * g4 + j;
                Ft0[jj * PF + i] = jj <= i ? (i == jj ? 1.f : 0.f) - t[j] : 0.f;
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
                zt[s] = mfma_kb1(ld4(Ft0 + (16 * I + r16) * PF + 16 * kb + 4 * g4),
                                 ld4(Fdte + (16 * J + r16) * PF + 16 * kb + 4 * g4), zt[s]);
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
    // dM = -strict_lower(Z TE^T): the M terms of dbeta and dgamma, W_N + W_N^T -> WS; W_A -> WA
#pragma unroll
    for (int s = 0; s < LPW; ++s) {
        const int l = wave + NW * s;
        if (l < NL) {
            int I, J;
            tile_of(l, I, J);
            f32x4 m = {0.f, 0.f, 0.f, 0.f};
            for (int kb = 0; kb <= J; ++kb)
                m = mfma_kb1(ld4(Fz + (16 * I + r16) * PF + 16 * kb + 4 * g4),
                             EL::tof(ld_frag<E>(TEs + (16 * J + r16) * PT + 16 * kb + 4 * g4)), m);
            const int jj = 16 * J + r16;
            float rb[4], rg[4], cg = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * I + 4 * g4 + j;
                const bool strict = jj < i;
                const float dm = strict ? -m[j] : 0.f;
                const float n = Nk[s][j];                        // 0 off the strict lower triangle
                const float dn = bet[i] * dm;
                rb[j] = dm * n;
                rg[j] = dn * n;
                cg += dn * n;
                if (strict) {
                    const E wn = EL::from_f(dn * Dk[s][j]);
                    WS[i * PT + jj] = wn;
                    WS[jj * PT + i] = wn;
                }
                if (jj == i) WS[i * PT + i] = EL::from_f(0.f);
                WA[i * PT + jj] = EL::from_f(jj <= i ? aA[s][j] : 0.f);
                if (jj < i) WA[jj * PT + i] = EL::from_f(0.f);      // the upper tiles
            }
            cg = sum_rows(cg);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                rb[j] = sum16(rb[j]);
                rg[j] = sum16(rg[j]);
            }
            if (r16 == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    atomicAdd(&dbet[16 * I + 4 * g4 + j], rb[j]);
                    atomicAdd(&dgam[16 * I + 4 * g4 + j], rg[j]);
                }
            }
            if (g4 == 0) atomicAdd(&dgam[jj], -cg);
        }
    }
    __syncthreads();

    // ---- dQ, dK of this wave's tiles, and their dgamma terms --------------
    {
        float rq[4] = {0.f, 0.f, 0.f, 0.f}, rx[4] = {0.f, 0.f, 0.f, 0.f}, re[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < JPW; ++s) {
            // q, k at rows 16 Iw + 4 g .. + 3 of column 16 (J0 + s) + r: one transpose read each
            const f32x4 qv = EL::tof(ld_colfrag<E>(Qs, PK, 16 * Iw, 16 * (J0 + s), lane));
            const f32x4 kv = EL::tof(ld_colfrag<E>(Ks, PK, 16 * Iw, 16 * (J0 + s), lane));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                rq[j] += qv[j] * aQ[s][j];
                rx[j] += kv[j] * aX[s][j];
                re[j] += kv[j] * aE[s][j];
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
    // 16-bit, C = 64: dQ, dK rows staged in LDS over N, dTE and Z (dead since the dM
    // step; the products below read only W_A, WS, K and Q), then written as
    // 16-byte units (the C layout gave two-byte stores: 10 us at gdn_340m)
    constexpr int PQ = DK + 8;
    constexpr bool STG = sizeof(E) == 2 && 2 * CH * PQ * (int)sizeof(E) <= 3 * CH * PF * 4;   // C = 64
    E *dQs = reinterpret_cast<E *>(R), *dKs = dQs + CH * PQ;
    const f32x4 GOr = ld4(go + 16 * Iw + 4 * g4), GXr = ld4(gx + 16 * Iw + 4 * g4), GEr = ld4(ge + 16 * Iw + 4 * g4);
#pragma unroll
    for (int s = 0; s < JPW; ++s) {
        const int J = J0 + s;
        f32x4 q = contract(aQ[s] * GOr, NB,
            [&](int kb) { return ld_frag<E>(WA + (16 * Iw + r16) * PT + 16 * kb + 4 * g4); },
            [&](int kb) { return ld_colfrag<E>(Ks, PK, 16 * kb, 16 * J, lane); });
        f32x4 k = contract(aE[s] * GEr - aX[s] * GXr, NB,
            [&](int kb) { return ld_colfrag<E>(WA, PT, 16 * kb, 16 * Iw, lane); },
            [&](int kb) { return ld_colfrag<E>(Qs, PK, 16 * kb, 16 * J, lane); });
        k = contract(k, NB,
            [&](int kb) { return ld_frag<E>(WS + (16 * Iw + r16) * PT + 16 * kb + 4 * g4); },
            [&](int kb) { return ld_colfrag<E>(Ks, PK, 16 * kb, 16 * J, lane); });
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = 16 * Iw + 4 * g4 + j;
            if constexpr (STG) {
                dQs[i * PQ + 16 * J + r16] = EL::from_f(q[j]);
                dKs[i * PQ + 16 * J + r16] = EL::from_f(k[j]);
            } else if (i < clen) {
                dqg[i * sqk + 16 * J + r16] = EL::from_f(q[j]);
                dkg[i * sqk + 16 * J + r16] = EL::from_f(k[j]);
            }
        }
    }
    __syncthreads();
    if constexpr (STG) {
        constexpr int VE = 16 / (int)sizeof(E), UPR = DK / VE;
        typedef E V __attribute__((ext_vector_type(VE)));
        for (int u = tid; u < CH * UPR; u += NT) {
            const int row = u / UPR, c0 = (u % UPR) * VE;
            if (row < clen) {
                *reinterpret_cast<V *>(dqg + row * sqk + c0) = *reinterpret_cast<const V *>(dQs + row * PQ + c0);
                *reinterpret_cast<V *>(dkg + row * sqk + c0) = *reinterpret_cast<const V *>(dKs + row * PQ + c0);
            }
        }
    }
    // ---- dg (suffix sums of dgamma; gamma_C is gamma at the last token) and dbeta
    if (wave == 0) {
        float x = lane < clen ? dgam[lane] : 0.f;
        if (lane == clen - 1) x += misc[1];
        x = wave_suffix(x);
        if (lane < clen) {
            if (p.dg) p.dg[(t0 + lane) * H + h] = x;
            const float b = bet[lane];                         // sigmoid(logit) when fused: its derivative b (1 - b)
            if (p.dbeta) p.dbeta[(t0 + lane) * H + h] = p.fz.beta_sigmoid ? dbet[lane] * b * (1.f - b) : dbet[lane];
        }
    }
}

// g per channel, or with the fused activation its pre-activation f (fp32, or
// the element type when Fusion::gate_16), at element offset off
template <typename E>
__device__ __forceinline__ float load_gate(const ChunkBwdParams &p, int64_t off) {
    if constexpr (sizeof(E) == 2)
        if (p.fz.gate_act && p.fz.gate_16) return Elem<E>::to_f(reinterpret_cast<const E *>(p.g)[off]);
    return p.g[off];
}

// ===========================================================================
// chunk_grad_vec_kernel: dQ, dK, dbeta, dg of one (chunk, head), per-channel gate
// ===========================================================================
// With the per-channel gate the CH x CH products are gated per key channel c,
// E_ij[c] = exp(gamma_i[c] - gamma_j[c]) (i >= j, so E <= 1):
//     N_ij = sum_c k_i[c] k_j[c] E_ij[c] (i > j)      A_ij = scale sum_c q_i[c] k_j[c] E_ij[c] (i >= j)
// and the other gated operands are the tiles K*G = k e^gamma, scale Q*G and
// K*Gend = k e^(gamma_C - gamma).  From dA, dTE and the dv sums the column phase
// left in p.gw (chunk_grad_kernel<VEC>) and N (chunk prep):
//     T0 = I - TE N,  Z = T0^T dTE,  dM = -strict_lower(Z TE^T),  dN = diag(beta) dM,
//     dbeta_i = Z_ii + sum_j dM_ij N_ij,   W_A = scale dA
//     SA_i = sum_{j<=i} W_A_ij k_j E_ij     SN_i = sum_{j<i} dN_ij k_j E_ij
//     TJ_j = sum_{i>=j} (W_A_ij q_i + dN_ij k_i) E_ij                      (per channel)
//     dq_i = SA_i + scale e^gamma_i (dO S^T)_i
//     dk_i = SN_i + TJ_i - e^gamma_i (dX S^T)_i + e^(gamma_C - gamma_i) (U dS'^T)_i
//     dgamma_i = q_i SA_i + k_i SN_i - k_i TJ_i
//                + (scale q e^gamma) (dO S^T) - (k e^gamma) (dX S^T) - (k e^(gamma_C - gamma)) (U dS'^T)
//     dgamma_C += sum_i (k e^(gamma_C - gamma))_i (U dS'^T)_i + e^gamma_C sum_cols S dS'
//     dg_t = dgamma_C + sum_{i >= t} dgamma_i
// SA, SN and TJ are MFMA products over 16-row blocks with one reference row
// per output block, as chunk prep builds N and A: for output rows in block I,
// E_ij = e^(gamma_i - gamma_r) e^(gamma_r - gamma_j) with r = 16 I (SA, SN) or
// r = 16 I + 15 (TJ), so that off the diagonal block both factors are <= 1.
// Every lane builds its own gated B fragments (its key channel c, rows
// 16 J + 4 g + 0..3) in registers.  The products run in fp32
// (v_mfma_f32_16x16x4f32; they are small): dgamma subtracts sums of like
// size (q SA against k TJ), which 16-bit operands would leave with a
// correlated error.  On a diagonal block the second factor reaches
// e^(gamma_16I - gamma_16I+15); a block whose range exceeds 60 nats on any
// channel takes exact per-pair exponentials there instead.  Wave w owns key-channel tile w % (DK / 16) and row blocks
// w / (DK / 16) + (8 / (DK / 16)) s; its MFMA output rows and column are the
// rows and channel whose q, k and gamma it holds, so the epilogue runs in
// registers.
// WR: explicit write vectors w in place of beta k (chunk prep's WR blocks:
// M_ij = <k_i, w_j>_E, A_ij = scale <q_i, w_j>_E, TE = (I + M)^-1, the write
// tile W*Gend).  beta is 1 (dN = dM), the j side of M and A is w, and the
// write tile's gradient goes to w:
//     SA_i = sum_j W_A_ij w_j E_ij     SN_i = sum_j dM_ij w_j E_ij     TJ as above (-> dw)
//     dk_i = SN_i - e^gamma_i (dX S^T)_i     dw_j = TJ_j + e^(gamma_C - gamma_j) (U dS'^T)_j
//     dgamma_i = q_i SA_i + k_i SN_i - w_i TJ_i + (scale q e^gamma) (dO S^T) - (k e^gamma) (dX S^T)
//                - (w e^(gamma_C - gamma)) (U dS'^T),  dgamma_C += sum_i (w e^(gamma_C - gamma))_i (U dS'^T)_i + ...
template <int DK, int CH, typename E, bool WR = false>
__global__ void __launch_bounds__(512) chunk_grad_vec_kernel(const ChunkBwdParams p) {
    using EL = Elem<E>;
    using CB = ChunkBlock<E, CH, DK, 2>;
    static_assert(CB::VEC && CH == 64, "per-channel gated tiles, 64-token chunks");
    constexpr int NT = 512, NW = 8, NB = CH / 16, NRG = NT / DK, RPT = CH / NRG;
    constexpr int FF = CH * CH, PW = CH + 4;                          // W pitch (floats)
    constexpr int NCT = DK / 16, WPC = NW / NCT, IPW = NB / WPC;   // channel tiles, waves per tile, blocks per wave
    static_assert(NT % DK == 0 && CH % NRG == 0 && NW % NCT == 0 && NB % WPC == 0, "thread layout");
    constexpr int VE = 16 / (int)sizeof(E), UPR = DK / VE, OUT_N = (CH * UPR + NT - 1) / NT;
    typedef E V __attribute__((ext_vector_type(VE)));
    __shared__ __attribute__((aligned(16))) E qs[CH * DK];          // q, later dq
    __shared__ __attribute__((aligned(16))) E ks[CH * DK];          // k, later dk
    __shared__ __attribute__((aligned(16))) E ws[WR ? CH * DK : 8]; // w, later dw (WR)
    __shared__ __attribute__((aligned(16))) float gms[CH * DK];     // gamma, later dgamma
    // TE (element type, as chunk prep wrote it), the CH x CH algebra's fp32
    // matrices (pitch PW), then (same memory) the A operands of the gated sums
    constexpr int PT = Pitch<E, CH>::value;
    constexpr int MM = CH * PW, NL = NB * (NB + 1) / 2, LPW = (NL + NW - 1) / NW;   // lower 16 x 16 tiles
    __shared__ __attribute__((aligned(16))) E tes[CH * PT];
    __shared__ __attribute__((aligned(16))) float alg[3 * MM];
    float *nn = alg, *b1 = alg + MM, *b2 = alg + 2 * MM;     // N, T0 then Z, dTE
    float *wa = alg, *wn = alg + MM;                         // W_A = scale dA (lower), dN (strict lower)
    __shared__ float bet[CH], dbet[CH], dgc[DK];
    __shared__ float part[NRG][DK];                          // per row group: sums of g, of dgamma, of df
    __shared__ float dbet_w[NW];                             // per wave: dA_log sums (fused activation)
    __shared__ int flag[NB];

    const int tid = threadIdx.x;
    const int c = tid % DK, rg = tid / DK;                   // channel phases
    const int H = p.H;
    const int h = blockIdx.x % H;
    const int64_t slot = blockIdx.x / H;
    int seq;
    int64_t cin;
    if (!locate_chunk(p.geo, slot, seq, cin)) return;
    int64_t bos, eos;
    seq_bounds(p.geo, seq, bos, eos);
    const int64_t t0 = bos + cin * CH;
    const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
    const int64_t sqk = (int64_t)H * DK;
    const char *blkb = reinterpret_cast<const char *>(p.blocks) + (slot * H + h) * CB::BYTES;
    const E *TEb = reinterpret_cast<const E *>(blkb);
    const float *nb = p.nbuf + (slot * H + h) * FF;
    const float *gwb = p.gw + (slot * H + h) * grad_vec_work_floats(CH, DK);
    const float *gQ = gwb, *gX = gwb + CH * DK, *gE = gwb + 2 * CH * DK;
    const float *gA = gwb + 3 * CH * DK, *gT = gA + FF, *gC = gT + FF;

    // ---- stage -------------------------------------------------------------
    constexpr int U4 = FF / 4 / NT;                          // 16-byte units of a CH x CH fp32 matrix per thread
    static_assert(FF % (4 * NT) == 0, "CH x CH units split evenly");
    f32x4 wav[U4];                                           // W_A units, stored after the algebra
    {
        BlockRegs<E, CH, NT> rte;
        rte.load(TEb, tid);
        f32x4 nv[U4], tv[U4];
#pragma unroll
        for (int m = 0; m < U4; ++m) {
            const int u = tid + NT * m;
            nv[m] = ld4(nb + 4 * u);
            tv[m] = ld4(gT + 4 * u);
            wav[m] = ld4(gA + 4 * u);
        }
        RowRegs<E, CH, DK, NT> rk, rq, rw;
        rk.load(reinterpret_cast<const E *>(p.k) + t0 * sqk + (int64_t)h * DK, sqk, clen, tid);
        rq.load(reinterpret_cast<const E *>(p.q) + t0 * sqk + (int64_t)h * DK, sqk, clen, tid);
        if constexpr (WR) rw.load(reinterpret_cast<const E *>(p.w) + t0 * sqk + (int64_t)h * DK, sqk, clen, tid);
        // gamma: inclusive sums over rows rg RPT .. + RPT - 1 here, the earlier groups' totals added below
        // (fused activation: g = act(f) from the pre-activation, as chunk prep computes it)
        float gv[RPT];
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const int i = rg * RPT + r;
            gv[r] = i < clen ? load_gate<E>(p, (t0 + i) * sqk + (int64_t)h * DK + c) : 0.f;
        }
        if (p.fz.gate_act) {
            const float a_log = p.fz.A_log[h], dt = p.fz.dt_bias[(int64_t)h * DK + c];
#pragma unroll
            for (int r = 0; r < RPT; ++r)
                gv[r] = rg * RPT + r < clen ? gate_activation(gv[r], a_log, dt, p.fz.lb_set, p.fz.lb) : 0.f;
        }
        rk.store(ks, DK, clen, tid);
        rq.store(qs, DK, clen, tid);
        if constexpr (WR) rw.store(ws, DK, clen, tid);
#pragma unroll
        for (int r = 1; r < RPT; ++r) gv[r] += gv[r - 1];
        part[rg][c] = gv[RPT - 1];
#pragma unroll
        for (int r = 0; r < RPT; ++r) gms[(rg * RPT + r) * DK + c] = gv[r];
        rte.store(tes, PT, tid);
#pragma unroll
        for (int m = 0; m < U4; ++m) {
            const int u = tid + NT * m, row = (4 * u) / CH, c0 = (4 * u) % CH;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                nv[m][e] = c0 + e < row ? nv[m][e] : 0.f;
                tv[m][e] = c0 + e <= row ? tv[m][e] : 0.f;
                wav[m][e] = c0 + e <= row ? p.scale * wav[m][e] : 0.f;
            }
            st4(nn + row * PW + c0, nv[m]);
            st4(b2 + row * PW + c0, tv[m]);
        }
        if (tid < CH) {
            const float b = WR ? 1.f : (tid < clen && p.beta ? p.beta[(t0 + tid) * H + h] : 0.f);   // no delta rule: 0
            bet[tid] = tid < clen ? (p.fz.beta_sigmoid ? sigmoidf_(b) : b) : 0.f;
            dbet[tid] = 0.f;
        }
        if (tid < DK) dgc[tid] = 0.f;
        if (tid < NB) flag[tid] = 0;
    }
    __syncthreads();
    if (rg > 0) {                                            // gamma: in-chunk inclusive sums, per channel
        float pre = 0.f;
        for (int r = 0; r < rg; ++r) pre += part[r][c];
#pragma unroll
        for (int r = 0; r < RPT; ++r) gms[(rg * RPT + r) * DK + c] += pre;
    }
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    auto tile_of = [](int l, int &I, int &J) __attribute__((always_inline)) {
        I = 0;
        J = l;
        while (J > I) { J -= I + 1; ++I; }
    };
    // T0 = I - TE N over the lower tiles (fp32 MFMA)
#pragma unroll
    for (int s = 0; s < LPW; ++s) {
        const int l = wave + NW * s;
        if (l < NL) {
            int I, J;
            tile_of(l, I, J);
            f32x4 t = {0.f, 0.f, 0.f, 0.f};
            for (int kb = J; kb <= I; ++kb)
                t = mfma_kb1(EL::tof(ld_frag<E>(tes + (16 * I + r16) * PT + 16 * kb + 4 * g4)),
                             col4(nn, PW, 16 * kb + 4 * g4, 16 * J + r16), t);
            const int jj = 16 * J + r16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 16 * I + 4 * g4 + j;
                b1[i * PW + jj] = jj <= i ? (i == jj ? 1.f : 0.f) - t[j] : 0.f;
            }
        }
    }
    __syncthreads();
    // blocks whose in-block decay range leaves the factorised form's limit
    if (rg == 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (gms[16 * b * DK + c] - gms[(16 * b + 15) * DK + c] > 60.f) flag[b] = 1;
    }
    // Z = T0^T dTE (lower tiles); dbeta_i += Z_ii
    {
        f32x4 zt[LPW];
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            zt[s] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int l = wave + NW * s;
            if (l < NL) {
                int I, J;
                tile_of(l, I, J);
                for (int kb = I; kb < NB; ++kb)
                    zt[s] = mfma_kb1(col4(b1, PW, 16 * kb + 4 * g4, 16 * I + r16),
                                     col4(b2, PW, 16 * kb + 4 * g4, 16 * J + r16), zt[s]);
                if (I == J) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (4 * g4 + j == r16) dbet[16 * I + r16] += zt[s][j];     // one lane per diagonal entry
                }
            }
        }
        __syncthreads();                                     // T0 and dTE are consumed
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            const int l = wave + NW * s;
            if (l < NL) {
                int I, J;
                tile_of(l, I, J);
#pragma unroll
                for (int j = 0; j < 4; ++j) b1[(16 * I + 4 * g4 + j) * PW + 16 * J + r16] = zt[s][j];
            }
        }
    }
    __syncthreads();
    // dM = -strict_lower(Z TE^T) (lower tiles); dbeta_i += sum_j dM_ij N_ij; dN = diag(beta) dM;
    // then W_A and dN replace the algebra's matrices
    {
        f32x4 dn[LPW];
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            dn[s] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int l = wave + NW * s;
            if (l < NL) {
                int I, J;
                tile_of(l, I, J);
                f32x4 m = {0.f, 0.f, 0.f, 0.f};
                for (int kb = 0; kb <= J; ++kb)
                    m = mfma_kb1(ld4(b1 + (16 * I + r16) * PW + 16 * kb + 4 * g4),
                                 EL::tof(ld_frag<E>(tes + (16 * J + r16) * PT + 16 * kb + 4 * g4)), m);
                const int jj = 16 * J + r16;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 16 * I + 4 * g4 + j;
                    const float dm = jj < i ? -m[j] : 0.f;
                    const float rb = sum16(dm * nn[i * PW + jj]);
                    if (r16 == 0) atomicAdd(&dbet[i], rb);
                    dn[s][j] = bet[i] * dm;
                }
            }
        }
        __syncthreads();                                     // Z and N are consumed
#pragma unroll
        for (int m = 0; m < U4; ++m) {
            const int u = tid + NT * m;
            st4(wa + ((4 * u) / CH) * PW + (4 * u) % CH, wav[m]);
        }
#pragma unroll
        for (int s = 0; s < LPW; ++s) {
            const int l = wave + NW * s;
            if (l < NL) {
                int I, J;
                tile_of(l, I, J);
#pragma unroll
                for (int j = 0; j < 4; ++j) wn[(16 * I + 4 * g4 + j) * PW + 16 * J + r16] = dn[s][j];
            }
        }
    }
    __syncthreads();

    // ---- the gated sums (MFMA) and the direct terms ----------------------------
    const int cc = 16 * (wave % NCT) + r16;                  // this lane's key channel
    float kr[NB][4], qr[NB][4], gr[NB][4];                   // rows 16 J + 4 g4 + jj of channel cc
    float wr[WR ? NB : 1][4];                                // (WR) w at the same rows
#pragma unroll
    for (int J = 0; J < NB; ++J)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int row = 16 * J + 4 * g4 + jj;
            kr[J][jj] = EL::to_f(ks[row * DK + cc]);
            qr[J][jj] = EL::to_f(qs[row * DK + cc]);
            gr[J][jj] = gms[row * DK + cc];
            if constexpr (WR) wr[J][jj] = EL::to_f(ws[row * DK + cc]);
        }
    const E *js = WR ? ws : ks;                              // the j side of M and A: w, or k
    const float gCc = gms[(CH - 1) * DK + cc];               // gamma_C (rows past the end add no decay)
    const float gCt = gms[(CH - 1) * DK + c];                // the same for the dg pass's channel
    // Each block's dq, dk (dw) and dgamma replace its q, k (w) and gamma in LDS as
    // soon as it is done: a lane reads and writes only its own channel there, and
    // after this point only the rows of its own blocks.  Where two waves share a
    // channel tile, the barrier keeps the writes behind both waves' loads above.
    if constexpr (WPC > 1) __syncthreads();
    float dgc_acc = 0.f;
#pragma unroll
    for (int s = 0; s < IPW; ++s) {
        const int I = wave / NCT + WPC * s;
        // rows 16 I + 4 g .. + 3 of key cc (the work area holds the sums transposed)
        f32x4 dqg = ld4(gQ + cc * CH + 16 * I + 4 * g4), dxs = ld4(gX + cc * CH + 16 * I + 4 * g4),
              dke = ld4(gE + cc * CH + 16 * I + 4 * g4);
        const bool exact = flag[I] != 0;                     // uniform over the workgroup
        const float gref = gms[16 * I * DK + cc], gend = gms[(16 * I + 15) * DK + cc];
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sn = sa, tj = sa;
        // SA, SN: B = k_j e^(gamma_r - gamma_j) over row blocks J <= I
#pragma unroll
        for (int J = 0; J < NB; ++J) {
            if (J < I || (J == I && !exact)) {
                f32x4 b;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) b[jj] = (WR ? wr[J][jj] : kr[J][jj]) * __expf(gref - gr[J][jj]);
                sa = mfma_kb1(ld4(wa + (16 * I + r16) * PW + 16 * J + 4 * g4), b, sa);
                sn = mfma_kb1(ld4(wn + (16 * I + r16) * PW + 16 * J + 4 * g4), b, sn);
            }
        }
        // TJ: B = (q_i, k_i) e^(gamma_i - gamma_r') over row blocks I2 >= I, A = W^T
#pragma unroll
        for (int I2 = 0; I2 < NB; ++I2) {
            if (I2 > I || (I2 == I && !exact)) {
                f32x4 bq, bk;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float e = __expf(gr[I2][jj] - gend);
                    bq[jj] = qr[I2][jj] * e;
                    bk[jj] = kr[I2][jj] * e;
                }
                tj = mfma_kb1(col4(wa, PW, 16 * I2 + 4 * g4, 16 * I + r16), bq, tj);
                tj = mfma_kb1(col4(wn, PW, 16 * I2 + 4 * g4, 16 * I + r16), bk, tj);
            }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const float gi = gr[I][jj];
            const float fa = __expf(gi - gref), ft = __expf(gend - gi);
            sa[jj] *= fa;
            sn[jj] *= fa;
            tj[jj] *= ft;
        }
        if (exact) {
            // the diagonal block with per-pair exponentials
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int i = 16 * I + 4 * g4 + jj;
                const float gi = gr[I][jj];
                float a = 0.f, n = 0.f, t = 0.f;
                for (int j = 16 * I; j <= i; ++j) {
                    const float kj = EL::to_f(js[j * DK + cc]) * __expf(gi - gms[j * DK + cc]);
                    a += wa[i * PW + j] * kj;
                    n += wn[i * PW + j] * kj;
                }
                for (int i2 = i; i2 < 16 * I + 16; ++i2) {
                    const float e = __expf(gms[i2 * DK + cc] - gi);
                    t += (wa[i2 * PW + i] * EL::to_f(qs[i2 * DK + cc]) + wn[i2 * PW + i] * EL::to_f(ks[i2 * DK + cc])) * e;
                }
                sa[jj] += a;
                sn[jj] += n;
                tj[jj] += t;
            }
        }
        // direct terms
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int i = 16 * I + 4 * g4 + jj;
            const float qi = qr[I][jj], ki = kr[I][jj], gi = gr[I][jj];
            const float eg = __expf(gi), egc = __expf(gCc - gi);
            dxs[jj] = p.delta ? dxs[jj] : 0.f;                 // without the delta rule K*G does not enter
            const bool ok = i < clen;
            float dkv, dgv;
            qs[i * DK + cc] = EL::from_f(ok ? sa[jj] + p.scale * eg * dqg[jj] : 0.f);
            if constexpr (WR) {
                const float wi = wr[I][jj];
                dkv = ok ? sn[jj] - eg * dxs[jj] : 0.f;
                ws[i * DK + cc] = EL::from_f(ok ? tj[jj] + egc * dke[jj] : 0.f);
                dgv = ok ? qi * sa[jj] + ki * sn[jj] - wi * tj[jj] + p.scale * qi * eg * dqg[jj] -
                               ki * eg * dxs[jj] - wi * egc * dke[jj]
                         : 0.f;
                dgc_acc += ok ? wi * egc * dke[jj] : 0.f;
            } else {
                dkv = ok ? sn[jj] + tj[jj] - eg * dxs[jj] + egc * dke[jj] : 0.f;
                dgv = ok ? qi * sa[jj] + ki * sn[jj] - ki * tj[jj] + p.scale * qi * eg * dqg[jj] -
                               ki * eg * dxs[jj] - ki * egc * dke[jj]
                         : 0.f;
                dgc_acc += ok ? ki * egc * dke[jj] : 0.f;
            }
            ks[i * DK + cc] = EL::from_f(dkv);
            gms[i * DK + cc] = dgv;
        }
    }
    atomicAdd(&dgc[cc], dgc_acc);
    __syncthreads();                                         // dq, dk (dw) and dgamma of every block are in LDS
    // dq, dk rows as 16-byte units
    {
        E *dqg = reinterpret_cast<E *>(p.dq) + t0 * sqk + (int64_t)h * DK;
        E *dkg = reinterpret_cast<E *>(p.dk) + t0 * sqk + (int64_t)h * DK;
        E *dwg = WR ? reinterpret_cast<E *>(p.dw) + t0 * sqk + (int64_t)h * DK : nullptr;
#pragma unroll
        for (int n = 0; n < OUT_N; ++n) {
            const int u = tid + n * NT;
            const int row = u / UPR, c0 = (u % UPR) * VE;
            if (u < CH * UPR && row < clen) {
                *reinterpret_cast<V *>(dqg + row * sqk + c0) = *reinterpret_cast<const V *>(qs + row * DK + c0);
                *reinterpret_cast<V *>(dkg + row * sqk + c0) = *reinterpret_cast<const V *>(ks + row * DK + c0);
                if constexpr (WR)
                    *reinterpret_cast<V *>(dwg + row * sqk + c0) = *reinterpret_cast<const V *>(ws + row * DK + c0);
            }
        }
    }
    // dg_t = dgamma_C + sum_{i >= t} dgamma_i, with dgamma_C = (the U dS'^T terms) + e^gamma_C sum S dS':
    // suffix sums over this thread's rows, then the later groups' totals
    float dv[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r) dv[r] = gms[(rg * RPT + r) * DK + c];
#pragma unroll
    for (int r = RPT - 2; r >= 0; --r) dv[r] += dv[r + 1];
    part[rg][c] = dv[0];
    __syncthreads();
    float post = dgc[c] + __expf(gCt) * gC[c];
    for (int r = rg + 1; r < NRG; ++r) post += part[r][c];
    if (p.fz.gate_act) {
        // through the activation: df = dg dg/dz (z = f + dt_bias), and this chunk's sums of
        // ddt_bias = sum_t df and dA_log = sum_{t, c} dg dg/dA_log
        //   softplus form g = -a sp(z), a = e^A_log:  dg/dz = -a sigmoid(z),  dg/dA_log = g
        //   bounded form  g = lb sigmoid(a z):        dg/dz = lb s (1 - s) a,  dg/dA_log = z dg/dz
        const float a_log = p.fz.A_log[h], dt = p.fz.dt_bias[(int64_t)h * DK + c], a = __expf(a_log);
        float sdt = 0.f, sda = 0.f;
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const int i = rg * RPT + r;
            if (i < clen) {
                const int64_t off = (t0 + i) * sqk + (int64_t)h * DK + c;
                const float z = load_gate<E>(p, off) + dt, dg = dv[r] + post;
                float dz, dA;
                if (p.fz.lb_set) {
                    const float s = sigmoidf_(a * z);
                    dz = p.fz.lb * s * (1.f - s) * a;
                    dA = dz * z;
                } else {
                    dz = -a * sigmoidf_(z);
                    dA = -a * softplusf_(z);
                }
                p.dg[off] = dg * dz;
                sdt += dg * dz;
                sda += dg * dA;
            }
        }
        __syncthreads();                                     // the suffix totals are read
        part[rg][c] = sdt;
        const float w = sum64(sda);
        if ((tid & 63) == 0) dbet_w[tid >> 6] = w;
        __syncthreads();
        float *dp = p.dpart + (slot * H + h) * (DK + 1);
        if (rg == 0) {
            float t = 0.f;
            for (int r = 0; r < NRG; ++r) t += part[r][c];
            dp[c] = t;
        }
        if (tid == 0) {
            float t = 0.f;
            for (int w8 = 0; w8 < NT / 64; ++w8) t += dbet_w[w8];
            dp[DK] = t;
        }
    } else if (p.dg) {
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            const int i = rg * RPT + r;
            if (i < clen) p.dg[(t0 + i) * sqk + (int64_t)h * DK + c] = dv[r] + post;
        }
    }
    if (tid < clen && p.dbeta) {
        const float b = bet[tid];                            // sigmoid(logit) when fused: its derivative b (1 - b)
        p.dbeta[(t0 + tid) * H + h] = p.fz.beta_sigmoid ? dbet[tid] * b * (1.f - b) : dbet[tid];
    }
}

// dA_log and dt_bias of the fused gate activation: the per-chunk sums
// chunk_grad_vec_kernel left, added over the chunks in slot order (one
// workgroup per head, a thread per dt_bias channel and one for A_log), so the
// result does not depend on scheduling
template <int DK>
__global__ void __launch_bounds__(256) gate_param_grad_kernel(const ChunkBwdParams p) {
    const int h = blockIdx.x, c = threadIdx.x;
    if (c > DK) return;
    int64_t n = p.geo.cu ? (int64_t)p.geo.chunk_offs[p.geo.n_seqs] : (int64_t)p.n_chunk_slots;
    n = n < p.n_chunk_slots ? n : p.n_chunk_slots;
    float acc = 0.f;
    for (int64_t s = 0; s < n; ++s) acc += p.dpart[(s * p.H + h) * (DK + 1) + c];
    if (c < DK) p.ddt_bias[(int64_t)h * DK + c] = acc;
    else p.dA_log[h] = acc;
}

// ===========================================================================
// launch
// ===========================================================================
template <int DK, int CH, typename E>
static hipError_t run_bwd(ChunkBwdParams p, bool saved, hipStream_t stream) {
    const int64_t units = (int64_t)p.geo.n_seqs * p.H;
    // Both walks take 32-column tiles (256 workgroups at B = 8, H = 8, dv =
    // 128) with two compute waves and producer waves (measured at B8 T4096 H8
    // d128, whole backward: 1.13 ms with the dS walk's compute waves staging
    // their own operands, 1.00 ms with producers; 1.02 ms with 64-column tiles).
    // The 16-bit dS walk runs four producers, each holding a quarter of a
    // chunk's operands in each of its two register sets (two producers: 256
    // VGPRs and 89 AGPRs; four: 162; gdn_340m backward 672 -> 661 us).
    if (units > 0) {
        p.n_tiles = (p.DV + 31) / 32;
        // 16-bit: the states came from the forward's state kernel (chunk_bwd), or a
        // training forward stored them
        if (!saved && sizeof(E) == 4)
            hipLaunchKernelGGL((chunk_hs_kernel<DK, CH, 2, E>), dim3((unsigned)((units + 7) / 8 * 8 * p.n_tiles)),
                               dim3(256), 0, stream, p);
        if constexpr (sizeof(E) == 2)
            hipLaunchKernelGGL((chunk_dhs_kernel<DK, CH, 2, E, false, 4>),
                               dim3((unsigned)((units + 7) / 8 * 8 * p.n_tiles)), dim3(384), 0, stream, p);
        else
            hipLaunchKernelGGL((chunk_dhs_kernel<DK, CH, 2, E>), dim3((unsigned)((units + 7) / 8 * 8 * p.n_tiles)),
                               dim3(256), 0, stream, p);
    }
    const int64_t grad_blocks = (int64_t)p.n_chunk_slots * p.H;
    if (grad_blocks > 0)
        hipLaunchKernelGGL((chunk_grad_kernel<DK, CH, E>), dim3((unsigned)grad_blocks), dim3(512), 0, stream, p);
    return hipGetLastError();
}

// Per-channel gate: the entry states come from the forward's state kernel
// (chunk_fwd with ChunkParams::hs), then the dS walk on the gated tiles, the
// column phase into p.gw and the per-channel gated gradients.
template <int DK, int CH, typename E>
static hipError_t run_bwd_vec(ChunkBwdParams p, hipStream_t stream) {
    const int64_t units = (int64_t)p.geo.n_seqs * p.H;
    if (units > 0) {
        // 32-column tiles once they give every CU a walk, 16-column tiles (one
        // compute wave, two producer waves) below that: the 128 dependent chunk
        // steps of a B4 T8192 H8 call ran on half the CUs with 32 columns
        if (units * ((p.DV + 31) / 32) >= device_cu_count()) {
            p.n_tiles = (p.DV + 31) / 32;
            hipLaunchKernelGGL((chunk_dhs_kernel<DK, CH, 2, E, true>), dim3((unsigned)((units + 7) / 8 * 8 * p.n_tiles)),
                               dim3(256), 0, stream, p);
        } else {
            p.n_tiles = (p.DV + 15) / 16;
            hipLaunchKernelGGL((chunk_dhs_kernel<DK, CH, 1, E, true, 2>),
                               dim3((unsigned)((units + 7) / 8 * 8 * p.n_tiles)), dim3(192), 0, stream, p);
        }
    }
    const int64_t grad_blocks = (int64_t)p.n_chunk_slots * p.H;
    if (grad_blocks > 0) {
        hipLaunchKernelGGL((chunk_grad_kernel<DK, CH, E, true>), dim3((unsigned)grad_blocks), dim3(512), 0, stream, p);
        if (p.w)
            hipLaunchKernelGGL((chunk_grad_vec_kernel<DK, CH, E, true>), dim3((unsigned)grad_blocks), dim3(512), 0,
                               stream, p);
        else
            hipLaunchKernelGGL((chunk_grad_vec_kernel<DK, CH, E>), dim3((unsigned)grad_blocks), dim3(512), 0, stream,
                               p);
        if (p.fz.gate_act)
            hipLaunchKernelGGL((gate_param_grad_kernel<DK>), dim3((unsigned)p.H), dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

hipError_t chunk_bwd(int dtype, int dk, int chunk, int gate_vector, const ChunkParams &fwd, ChunkBwdParams p,
                     int32_t *table, bool saved, hipStream_t stream) {
    if (p.geo.n_seqs == 0) return hipSuccess;
    const bool vec = gate_vector != 0;
    if (vec && (dtype == 0 || chunk != 64 || !fwd.hs || !fwd.nout || !p.nbuf || !p.gw))
        return hipErrorInvalidValue;                           // the per-channel backward: 16-bit, 64-token chunks
    if (p.fz.qk_l2norm || (p.fz.gate_act && (!vec || !p.dpart || !p.dA_log || !p.ddt_bias || !p.dg)))
        return hipErrorInvalidValue;
    // TE, A and the gate factors of every chunk, as the forward built them
    // (already in the workspace after a saving forward); with 16-bit elements
    // the forward's state kernel, run for the entry states alone (no outputs),
    // also walks the chunks (fp32: chunk_hs_kernel, in run_bwd)
    if (!saved) {
        ChunkParams f = fwd;
        const bool walk = dtype != 0;
        if (walk) {
            f.hs = p.hs;
            f.h0 = p.h0;
            f.states_only = 1;
        }
        hipError_t e = chunk_fwd(dtype, dk, chunk, vec ? 1 : 0, f, table, walk ? CHUNK_PREP | CHUNK_STATE : CHUNK_PREP,
                                 stream);
        if (e != hipSuccess) return e;
    }
    if (p.geo.cu) {
        p.geo.chunk_offs = table + 2 * p.geo.n_seqs;
        p.geo.order = table + 3 * p.geo.n_seqs + 1;
    }
    if (vec) {
        if (dtype == 1) {
            if (dk == 64) return run_bwd_vec<64, 64, __bf16>(p, stream);
            return run_bwd_vec<128, 64, __bf16>(p, stream);
        }
        if (dk == 64) return run_bwd_vec<64, 64, _Float16>(p, stream);
        return run_bwd_vec<128, 64, _Float16>(p, stream);
    }
#define VGDR_BWD(DK_, CH_, E_) return run_bwd<DK_, CH_, E_>(p, saved, stream);
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

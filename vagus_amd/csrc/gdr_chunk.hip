// Chunkwise prefill of the gated delta rule (GDN scalar gate, KDA
// per-channel gate, optional delta rule) for gfx950, as two kernels.
//
// Math (linear_attention.py:237-309 scalar, :312-425 per channel), in the
// unified per-channel form.  Per chunk of CH tokens with cumulative log decay
// gamma (a scalar per token for GDN, a DK-vector for KDA), G_i = exp(gamma_i),
// Gend_i = exp(gamma_C - gamma_i), Gc = exp(gamma_C):
//     M_ij = beta_i <k_i, k_j>_g   (j < i)         A_ij = scale <q_i, k_j>_g   (j <= i)
//     TE   = (I + M)^-1 diag(beta)
//     X    = V - (K*G) S                           (the WY form's U - W S, refactored:
//     U~   = TE X                                   W = TE (K*G), U = TE V)
//     o    = scale (Q*G) S + A U~
//     S   <- Gc (.) S + (K*Gend)^T U~
// with <x_i, y_j>_g = sum_c x_i[c] y_j[c] exp(gamma_i[c] - gamma_j[c]).
//
// chunk_prep_kernel  (one workgroup per (chunk, head); no dependence between
//     chunks, so the whole batch runs in parallel at high occupancy) builds the
//     state-independent TE and A of every chunk and stores them in MFMA
//     fragment order (see frag_pos).
// chunk_state_kernel (one workgroup per (sequence, head, 16*NW-column dv
//     tile)) walks the chunks in order.  Wave w owns 16 state columns and keeps
//     them in fp32 MFMA accumulators (C layout) for the whole sequence; the
//     products above run register-to-register.  The next chunk's operands
//     (K, Q, V rows, TE and A) are copied global -> LDS asynchronously into the
//     other half of a double buffer while the current chunk computes.
//
// Per-channel gates reach the MFMA through a sub-block factorisation: for
// token blocks I >= J of 16 and reference row r = 16 I,
//     exp(gamma_i - gamma_j) = exp(gamma_i - gamma_r) * exp(gamma_r - gamma_j).
// Off-diagonal blocks (j < r <= i) have both exponents <= 0.  A diagonal
// block's second factor is >= 1, bounded by the block's own decay range; a
// block whose range exceeds Elem<E>::gate_range nats takes an exact pairwise
// path instead, so no overflowing exponential is ever formed.
#include "gdr_chunk_layout.hpp"
#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

// ---------------------------------------------------------------------------
// LDS tiles written by the asynchronous global->LDS path
// ---------------------------------------------------------------------------
// A row-major tile of NCOL-element rows stored without padding; its 16-byte
// units are XOR-swizzled within each row (unit c of row r sits at unit
// position c ^ (r % UPR)), so that the fragment reads of 16 consecutive rows
// at one column spread over all LDS banks.
// global -> LDS copies of 16 / 4 bytes per lane: lane L writes LDS base + L * size
// (global_load_lds_dword{,x4}; the LDS base goes in M0).  Written as inline asm
// on purpose: the compiler then does not know that the instruction writes LDS,
// so it never makes later LDS reads of the *other* double-buffer slot wait for
// the copy.  Completion is managed explicitly: dma_wait() (s_waitcnt vmcnt(0))
// by every issuing wave, then a barrier, before any lane reads the slot; the
// memory clobber keeps the compiler from moving LDS accesses across the copy.
// M0 is set inside the asm and is otherwise unused by these kernels (no
// movrel / LDS-parameter instructions), so clobbering it is safe here.  An
// LDS DMA that reads M0 needs one wait state after the SALU write of M0
// (a GFX9-family hazard), hence the s_nop between the two.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void *src, void *lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr(lds_base))) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void *src, void *lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :: "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr(lds_base))) : "memory", "m0");
}
#pragma clang diagnostic pop

template <typename E, int NCOL>
struct Swz {
    static constexpr int VE = 16 / sizeof(E);
    static constexpr int UPR = NCOL / VE;                     // 16-byte units per row
    static_assert((UPR & (UPR - 1)) == 0, "units per row must be a power of two");
    __device__ static __forceinline__ int at(int r, int c) {
        return r * NCOL + (((c / VE) ^ (r & (UPR - 1))) * VE) + (c & (VE - 1));
    }
};

// Issue the asynchronous copy of rows [0, CH) x columns [0, NCOL) of a token-
// major global matrix (row r at src + r * stride) into a swizzled LDS tile.
// Rows >= valid_rows and columns >= valid_cols are zero-filled with ordinary
// LDS stores instead.  global_load_lds writes lane L's 16 bytes at the
// wave-uniform LDS base + 16 L, so each wave fills 64 consecutive units and the
// swizzle is applied by choosing which global unit each lane fetches.
// Completion: s_waitcnt vmcnt(0) by the issuing wave, then a barrier.
template <typename E, int CH, int NCOL, int NT, bool SWIZZLE = true>
__device__ __forceinline__ void dma_rows(E *lds, const E *src, int64_t stride, int valid_rows, int valid_cols,
                                int tid) {
    using S = Swz<E, NCOL>;
    constexpr int UNITS = CH * S::UPR;
    constexpr int NWV = NT / 64;
    static_assert(UNITS % NT == 0, "tile does not split evenly over the workgroup");
    const int wave = tid >> 6, lane = tid & 63;
    // zero-fill first: an ordinary LDS store issued after a DMA into the same
    // array would make the compiler wait for that DMA
#pragma unroll
    for (int i = 0; i < UNITS / NT; ++i) {
        const int u = (wave + NWV * i) * 64 + lane;
        const int r = u / S::UPR, pp = u % S::UPR;
        const int c = SWIZZLE ? (pp ^ (r & (S::UPR - 1))) : pp;
        if (!(r < valid_rows && c * S::VE < valid_cols))
            *reinterpret_cast<Vec16 *>(lds + u * S::VE) = Vec16{{0u, 0u, 0u, 0u}};
    }
#pragma unroll
    for (int i = 0; i < UNITS / NT; ++i) {
        const int wu = (wave + NWV * i) * 64;                 // first unit of this wave's run
        const int u = wu + lane;
        const int r = u / S::UPR, pp = u % S::UPR;
        const int c = SWIZZLE ? (pp ^ (r & (S::UPR - 1))) : pp;
        if (r < valid_rows && c * S::VE < valid_cols)
            lds_dma16(src + (int64_t)r * stride + c * S::VE, lds + wu * S::VE);
    }
}

// The same copy through registers: load() issues every 16-byte load of the
// tile at once (unconditionally, from a clamped address: a load under a
// per-lane branch gets a full wait in front of the next one), store() writes
// the swizzled LDS tile, zeros outside [valid_rows, valid_cols).  Measured on
// MI355X with every CU streaming, plain loads move several times more bytes
// per CU than global_load_lds.
template <typename E, int CH, int NCOL, int NT>
struct RegRows {
    using S = Swz<E, NCOL>;
    static constexpr int UNITS = CH * S::UPR, PER = UNITS / NT, NWV = NT / 64;
    static_assert(UNITS % NT == 0 && PER <= 32, "tile does not split evenly over the workgroup");
    u32x4 r[PER];
    uint32_t ok;
    __device__ __forceinline__ void load(const E *src, int64_t stride, int valid_rows, int valid_cols, int tid) {
        const int wave = tid >> 6, lane = tid & 63;
        ok = 0;
        unroll<PER>([&](auto i) {
            const int u = (wave + NWV * (int)i) * 64 + lane;
            const int row = u / S::UPR, pp = u % S::UPR, c = pp ^ (row & (S::UPR - 1));
            const bool in = row < valid_rows && c * S::VE < valid_cols;
            r[i] = *reinterpret_cast<const u32x4 *>(src + (in ? (int64_t)row * stride + c * S::VE : 0));
            ok |= (uint32_t)in << (int)i;
        });
    }
    __device__ __forceinline__ void store(E *lds, int tid) const {
        const int wave = tid >> 6, lane = tid & 63;
        unroll<PER>([&](auto i) {
            const int u = (wave + NWV * (int)i) * 64 + lane;
            *reinterpret_cast<u32x4 *>(lds + u * S::VE) = (ok >> (int)i) & 1u ? r[i] : u32x4{0u, 0u, 0u, 0u};
        });
    }
    // Scales every row to unit L2 norm, x rsqrt(sum x^2 + 1e-6) rounded to E
    // (linear_attention.py:703-706), and writes each row's factor to rf[row].
    // A row's UPR units sit in UPR consecutive lanes of one load.
    __device__ __forceinline__ void l2norm_rows(float *rf, int tid) {
        static_assert(sizeof(E) == 2 && 64 % S::UPR == 0, "rows of 16-bit elements within one wavefront");
        using V8 = typename Elem<E>::frag2;
        const int wave = tid >> 6, lane = tid & 63;
        unroll<PER>([&](auto i) {
            V8 x = __builtin_bit_cast(V8, r[i]);
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += (float)x[e] * (float)x[e];
#pragma unroll
            for (int off = 1; off < S::UPR; off <<= 1) ss += __shfl_xor(ss, off);
            const float f = rsqrtf(ss + 1e-6f);
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = (E)((float)x[e] * f);
            r[i] = __builtin_bit_cast(u32x4, x);
            const int u = (wave + NWV * (int)i) * 64 + lane;
            if (u % S::UPR == 0) rf[u / S::UPR] = f;
        });
    }
};

// contiguous copy of n16 16-byte units (identity layout)
template <typename E, int NUNITS, int NT>
__device__ __forceinline__ void dma_flat(E *lds, const E *src, int tid) {
    constexpr int VE = 16 / sizeof(E);
    static_assert(NUNITS % NT == 0, "block does not split evenly over the workgroup");
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int i = 0; i < NUNITS / NT; ++i) {
        const int wu = (wave + (NT / 64) * i) * 64;
        lds_dma16(src + (wu + lane) * VE, lds + wu * VE);
    }
}

__device__ __forceinline__ void dma_wait() { __builtin_amdgcn_s_waitcnt(0); }


// ===========================================================================
// chunk_prep_kernel: per (chunk, head) TE and A
// ===========================================================================
// the 16x16x32 operand type of a 16-bit element (a placeholder otherwise)
template <typename EL, bool B> struct Frag2Of { using type = f32x4; };
template <typename EL> struct Frag2Of<EL, true> { using type = typename EL::frag2; };

template <int DK, int CH, typename E, int GATE, bool WR = false>
struct PrepLayout {
    static constexpr int PF = CH + 4, PG = DK + 4;
    static constexpr int NL = (CH / 16) * (CH / 16 + 1) / 2;      // lower tile pairs
    // Per-channel gate: Q rows are not staged and the cumulative decay sits
    // after the K (W) stage; with 16-bit elements (FAST) the products' gated
    // operands, built once per row, then replace both (GTILES).  M, T reuse it
    // all: 53 KB at dk = 128, C = 64, three workgroups per CU instead of two
    // (measured: the kernel's time follows its occupancy, 218 us at one
    // workgroup per CU, 137 at two).
    // Scalar gate or none, 16-bit, C = 64 (LEAN): each wave owns one row block
    // and takes its Q rows as MFMA operands straight from global memory (no Q
    // stage); M and T are kept as their lower 16x16 tiles; A and M are written
    // as each product finishes, M into a region of its own, and T then reuses
    // the K stage.  29 KB at dk = 128 (35 KB before): five workgroups per CU
    // (measured at gdn_340m: 47.8 -> 45.1 us; six, with M held in registers
    // until the barrier and 26 KB, ran no faster and lengthened every
    // workgroup's loads).
    static constexpr bool LEAN = GATE != 2 && sizeof(E) == 2 && CH == 64 && !WR;
    static constexpr int TP = 20;                                  // LEAN: row pitch of a lower tile (floats)
    static constexpr int MT = NL * 16 * TP * 4;                    // LEAN: one matrix as lower tiles
    static constexpr bool QREG = GATE == 2 || LEAN;
    static constexpr bool FAST = GATE == 2 && sizeof(E) == 2;
    static constexpr int STAGE = ((WR ? 2 : 1) + (QREG ? 0 : 1)) * CH * DK * (int)sizeof(E);  // K (Q, W) rows, swizzled
    static constexpr int GAMB = GATE == 2 ? CH * PG * 4 : 0;      // cumulative decay per channel
    static constexpr int NORM = GATE == 2 ? 2 * CH * 4 : 0;       // rows' L2-norm factors of K, Q
    static constexpr int GTILES = FAST ? 3 * CH * DK * (int)sizeof(E) + NL * DK * 4 : 0;  // Qh, Kh, Kt, pair factors
    static constexpr int MOFF = LEAN ? cmax(STAGE, MT) : 0;        // byte offset of M (LEAN: past the stage)
    static constexpr int SOLVE = LEAN ? MOFF + MT : 2 * CH * PF * 4;  // M, T
    static constexpr int UNION = cmax(cmax(STAGE + GAMB + NORM, GTILES), SOLVE);
};

// WR: an explicit write vector w_t in place of beta_t k_t (the asymmetric
// delta rule, linear_attention.py:340-353, :389-396), per-channel gate only.
// W rows take the writing slot: M_ij = <k_i, w_j>_g, A_ij = scale <q_i, w_j>_g,
// TE = (I + M)^-1 (no beta), and the third gated tile is W * Gend; the state
// kernel is the per-channel one, unchanged.
template <int DK, int CH, typename E, int GATE, bool WR = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(
    GATE == 2 && DK == 128 && !WR ? 3 : (PrepLayout<DK, CH, E, GATE, WR>::LEAN ? 5 : 1))))
chunk_prep_kernel(const ChunkParams p) {
    static_assert(!WR || GATE == 2, "the explicit write runs on the per-channel-gate path");
    using EL = Elem<E>;
    using F = typename EL::frag;
    using L = PrepLayout<DK, CH, E, GATE, WR>;
    using SK = Swz<E, DK>;
    constexpr int NT = 256, NW = 4, NB = CH / 16, NKB = DK / 16, PF = L::PF, PG = L::PG;
    constexpr int NL = NB * (NB + 1) / 2;
    // tile jobs (I, J), J <= I.  With one row block per wave (CH = 64, scalar
    // gate), wave w takes row block I = w and its tiles J = 0..w: it reads its
    // Q_I, K_I fragments once instead of once per tile (40% fewer LDS reads in
    // the products).  The per-channel gate keeps the round-robin: its tiles
    // carry per-element exponentials, and the 4-tile wave of the row-block
    // split lengthened the phase (measured: 16k -> 18k cycles, plus the others'
    // wait at the barrier).  Otherwise the NL tiles go round-robin over the waves.
    constexpr bool RB = NB == NW && GATE != 2;
    constexpr int JPW = RB ? NB : (NL + NW - 1) / NW;           // tile jobs per wave

    __shared__ __attribute__((aligned(16))) char smem[L::UNION];
    __shared__ __attribute__((aligned(16))) float gam_s[GATE == 2 ? 4 : CH];
    __shared__ __attribute__((aligned(16))) float bet[CH];
    __shared__ __attribute__((aligned(16))) float rkf_s[GATE == 2 ? 4 : CH];  // rows' L2-norm factors (fused norm)
    __shared__ __attribute__((aligned(16))) float rqf_s[GATE == 2 ? 4 : CH];
    __shared__ int flag[4];
    E *Kst = reinterpret_cast<E *>(smem);
    E *Qst = L::QREG ? nullptr : Kst + CH * DK;
    E *Wst = WR ? Kst + CH * DK : Kst;                          // the writing slot: W rows, or K
    float *gam = GATE == 2 ? reinterpret_cast<float *>(smem + L::STAGE) : gam_s;
    float *rkf = GATE == 2 ? reinterpret_cast<float *>(smem + L::STAGE + L::GAMB) : rkf_s;
    float *rqf = GATE == 2 ? rkf + CH : rqf_s;
    // M and T after the products are done (LEAN: M from the products on);
    // mpos(I, J, r, c): element (16 I + r, 16 J + c) of a lower tile, rows RS apart
    float *Mf = reinterpret_cast<float *>(smem + L::MOFF);
    float *Tf = L::LEAN ? reinterpret_cast<float *>(smem) : Mf + CH * PF;
    constexpr int RS = L::LEAN ? L::TP : PF;
    auto mpos = [](int I, int J, int r, int c) __attribute__((always_inline)) {
        if constexpr (L::LEAN) return ((I * (I + 1) / 2 + J) * 16 + r) * L::TP + c;
        else return (16 * I + r) * PF + 16 * J + c;
    };

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    const int H = p.H;
    const int h = blockIdx.x % H;
    const int64_t slot = blockIdx.x / H;

    // ---- which chunk ------------------------------------------------------
    int seq;
    int64_t cin;
    if (p.geo.cu) {
        const int32_t *offs = p.geo.chunk_offs;
        if (slot >= offs[p.geo.n_seqs]) return;               // beyond the last chunk
        int lo = 0, hi = p.geo.n_seqs - 1;                     // largest s with offs[s] <= slot
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (offs[mid] <= slot) lo = mid; else hi = mid - 1;
        }
        seq = lo;
        cin = slot - offs[lo];
    } else {
        seq = (int)(slot / p.geo.chunks_per_seq);
        cin = slot % p.geo.chunks_per_seq;
        if (seq >= p.geo.n_seqs) return;
    }
    int64_t bos, eos;
    seq_bounds(p.geo, seq, bos, eos);
    const int64_t t0 = bos + cin * CH;
    const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
    const int64_t sqk = (int64_t)H * DK;
    const E *kg = reinterpret_cast<const E *>(p.k) + t0 * sqk + (int64_t)h * DK;
    const E *qg = reinterpret_cast<const E *>(p.q) + t0 * sqk + (int64_t)h * DK;
    using CB = ChunkBlock<E, CH, DK, GATE>;
    char *blk_base = reinterpret_cast<char *>(p.blocks) + (slot * H + h) * CB::BYTES;
    E *blk = reinterpret_cast<E *>(blk_base);                                    // TE, then A

    // ---- stage: gate and beta first (the scans wait for them), then K, Q rows
    // Every load is unconditional, from a clamped row, and all are in flight
    // together; rows past the end are zeroed afterwards.
    float beta_v = 0.f, g_v = 0.f;
    if (wave == 0) {
        const int row = lane < clen ? lane : 0;
        if (!WR && p.use_delta && !p.te_identity) beta_v = p.beta[(t0 + row) * H + h];
        if constexpr (GATE != 2)
            if (p.g) g_v = p.g[(t0 + row) * H + h];
    }
    const Fusion &fz = p.fz;
    // per-channel gate: thread (sg, cg) holds channels 4 cg .. + 3 of rows
    // RPS sg .. + RPS - 1
    constexpr int CG = DK / 4, SGN = NT / CG, RPS = CH / SGN;
    static_assert(GATE != 2 || (SGN * CG == NT && RPS * SGN == CH), "gate tile does not split over the workgroup");
    const int cg = tid % CG, sg = tid / CG;
    f32x4 gv[GATE == 2 ? RPS : 1];
    if constexpr (GATE == 2) {
        unroll<RPS>([&](auto i) {
            const int row = sg * RPS + (int)i, rr = row < clen ? row : 0;
            const int64_t off = ((t0 + rr) * H + h) * DK + 4 * cg;
            if constexpr (sizeof(E) == 2) {
                if (fz.gate_16) {                               // pre-activation f in the element type
                    const uint2 raw = *reinterpret_cast<const uint2 *>(reinterpret_cast<const E *>(p.g) + off);
                    gv[i] = EL::tof(__builtin_bit_cast(F, raw));
                } else {
                    gv[i] = ld4(p.g + off);
                }
            } else {
                gv[i] = ld4(p.g + off);
            }
        });
    }
    RegRows<E, CH, DK, NT> rk, rq;
    RegRows<E, CH, DK, NT> rw;                                  // W rows (WR only)
    rk.load(kg, sqk, clen, DK, tid);
    if constexpr (WR)
        rw.load(reinterpret_cast<const E *>(p.w) + t0 * sqk + (int64_t)h * DK, sqk, clen, DK, tid);
    // LEAN: this wave's Q rows 16 wave + r, as operands of 16x16x32 products whose
    // k slots are 32 m + 8 g .. + 7 (16-byte loads; rows past the end zeroed below)
    using V8 = typename Frag2Of<EL, L::LEAN>::type;
    V8 qfr[L::LEAN ? NKB / 2 : 1];
    if constexpr (L::LEAN) {
        const int qrow = 16 * wave + r16;
        const E *qsrc = qg + (int64_t)(qrow < clen ? qrow : 0) * sqk + 8 * g4;
#pragma unroll
        for (int m = 0; m < NKB / 2; ++m) qfr[m] = *reinterpret_cast<const V8 *>(qsrc + 32 * m);
    } else {
        rq.load(qg, sqk, clen, DK, tid);
    }
    if (wave == 0 && lane < CH)
        bet[lane] = lane < clen ? (WR ? 1.f : (fz.beta_sigmoid ? sigmoidf_(beta_v) : beta_v)) : 0.f;
    if constexpr (GATE == 2) {
        if (fz.gate_act) {                                      // g = act(f + dt_bias) per channel
            const float a_log = fz.A_log[h];
            const f32x4 dt = ld4(fz.dt_bias + (int64_t)h * DK + 4 * cg);
            unroll<RPS>([&](auto i) {
#pragma unroll
                for (int e = 0; e < 4; ++e) gv[i][e] = gate_activation(gv[i][e], a_log, dt[e], fz.lb_set, fz.lb);
            });
        }
        // inclusive cumulative sum over rows: within the thread's rows in
        // registers, then the totals of the preceding row segments from LDS
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        unroll<RPS>([&](auto i) {
            if (sg * RPS + (int)i < clen) acc += gv[i];
            gv[i] = acc;
        });
        // segment totals in the K stage, free until K and Q are stored below
        f32x4 *gtot = reinterpret_cast<f32x4 *>(Kst);
        gtot[sg * CG + cg] = acc;
        if (tid < 4) flag[tid] = 0;
        __syncthreads();
        f32x4 off = {0.f, 0.f, 0.f, 0.f};
        for (int s2 = 0; s2 < sg; ++s2) off += gtot[s2 * CG + cg];
        unroll<RPS>([&](auto i) { st4(gam + (sg * RPS + (int)i) * PG + 4 * cg, gv[i] + off); });
        __syncthreads();
        for (int it = tid; it < NB * DK; it += NT) {
            const int b = it / DK, c2 = it % DK;
            if (gam[(16 * b) * PG + c2] - gam[(16 * b + 15) * PG + c2] > EL::gate_range) flag[b] = 1;
        }
    } else {
        if (wave == 0) {
            const float x = wave_scan(lane < clen ? g_v : 0.f);
            if (lane < CH) gam[lane] = x;
        }
    }
    if constexpr (sizeof(E) == 2) {
        if (fz.qk_l2norm) {                                     // normalised rows, factors in rkf / rqf
            rk.l2norm_rows(rkf, tid);
            if constexpr (L::LEAN) {
                // the row's sum of squares over its four lanes (l, l ^ 16, l ^ 32, l ^ 48)
                float ss = 0.f;
#pragma unroll
                for (int m = 0; m < NKB / 2; ++m)
#pragma unroll
                    for (int e = 0; e < 8; ++e) ss += (float)qfr[m][e] * (float)qfr[m][e];
                ss += __shfl_xor(ss, 16);
                ss += __shfl_xor(ss, 32);
                const float f = rsqrtf(ss + 1e-6f);
#pragma unroll
                for (int m = 0; m < NKB / 2; ++m)
#pragma unroll
                    for (int e = 0; e < 8; ++e) qfr[m][e] = (E)((float)qfr[m][e] * f);
                if (g4 == 0) rqf[16 * wave + r16] = f;
            } else {
                rq.l2norm_rows(rqf, tid);
            }
        }
    }
    // ---- per-channel gate, 16-bit: one pass over the thread's K, Q (W) units
    // (unit i: global column unit c of row `row`, the swizzled load order) writes
    // the state kernel's gated tiles, K*G and K*Gend (W*Gend) in paired-column
    // order (16-byte unit pu = 4 q + g holds columns 32 q + 4 g .. + 3 and
    // 32 q + 16 + 4 g .. + 3) and scale Q*G in natural order, and forms the
    // products' operands with one exponential per (row, channel), relative to
    // the first row a = 16 I of the row's block:
    //   Qh = q e^(g - g_a), Kh = k e^(g - g_a)  (<= 1),  Kt = k e^(g_a - g)  (w with WR;
    //   at most e^gate_range when no block is flagged),
    // and per tile pair (I, J) the channel factors PF_IJ = e^(g_16I - g_16J)
    // (<= 1; 1 for J = I), so that the pair contracts Qh_i, Kh_i with
    // Kt_j * PF_IJ = k_j e^(g_16I - g_j) exactly as the per-pair factorisation
    // does, with no row after i involved (the diagonal tiles are those products
    // themselves; the others take one more rounding).  Rows past the end are
    // zero.  A chunk with a flagged block (range above gate_range) runs the
    // per-pair exponentials on the decay table instead.
    constexpr int UPR = SK::UPR, PER = decltype(rk)::PER, NPF = (L::NL * DK + NT - 1) / NT;
    u32x4 oq[L::FAST ? PER : 1], ok_[L::FAST ? PER : 1];
    float opf[L::FAST ? NPF : 1];
    bool fast = false;
    if constexpr (L::FAST) {
        using V8 = typename EL::frag2;
        E *tg = reinterpret_cast<E *>(blk_base) + CB::TEA;
        // LDS of the fast path: Kt over the K stage (free now), then Qh, Kh and the
        // pair factors over the decay table once every thread has read it
        E *Kt = reinterpret_cast<E *>(smem), *Qh = Kt + CH * DK, *Kh = Qh + CH * DK;
        float *PFs = reinterpret_cast<float *>(smem + 3 * CH * DK * (int)sizeof(E));
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
        // the thread's units lie in rows r0 + (NT / UPR) i and share one column
        // unit c, so gamma_C is read once; each unit runs in two halves of four
        // channels
        static_assert(64 % UPR == 0 && (NT / UPR) % UPR == 0, "units of one thread share their column unit");
        const int c = (lane % UPR) ^ (((wave * 64 + lane) / UPR) & (UPR - 1));
        f32x4 gC[2];
        gC[0] = ld4(gam + (CH - 1) * PG + 8 * c);
        gC[1] = ld4(gam + (CH - 1) * PG + 8 * c + 4);
        unroll<PER>([&](auto i) {
            const int u = (wave + (NT / 64) * (int)i) * 64 + lane;
            const int row = u / UPR, ra = row & ~15;
            const bool ok = (rk.ok >> (int)i) & 1u;
            const V8 xk = __builtin_bit_cast(V8, rk.r[(int)i]), xq = __builtin_bit_cast(V8, rq.r[(int)i]);
            V8 xw;
            if constexpr (WR) xw = __builtin_bit_cast(V8, rw.r[(int)i]);
            else xw = xk;
            F hq[2], hk[2], hqg[2];
            char *rowb = reinterpret_cast<char *>(tg + row * DK);
            // paired-order byte offset of the unit's first 4-column piece (the second: + 16)
            const int pb = 16 * (4 * (c >> 2) + 2 * (c & 1)) + 8 * ((c & 3) >> 1);
            unroll<2>([&](auto hh) {
                const int cc = 8 * c + 4 * (int)hh;
                const f32x4 g = ld4(gam + row * PG + cc), a = ld4(gam + ra * PG + cc);
                f32x4 k, q, w;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    k[e] = ok ? (float)xk[4 * (int)hh + e] : 0.f;
                    q[e] = ok ? (float)xq[4 * (int)hh + e] : 0.f;
                    w[e] = ok ? (float)xw[4 * (int)hh + e] : 0.f;
                }
                const f32x4 eg = exp4(g), ed = exp4(gC[(int)hh] - g), ea = exp4(g - a), eb = exp4(a - g);
                *reinterpret_cast<F *>(rowb + pb + 16 * (int)hh) = EL::cvt(p.te_identity ? f32x4{0.f, 0.f, 0.f, 0.f} : k * eg);
                hqg[(int)hh] = EL::cvt(q * eg * p.scale);
                *reinterpret_cast<F *>(rowb + 2 * CH * DK * (int)sizeof(E) + pb + 16 * (int)hh) = EL::cvt(w * ed);
                hq[(int)hh] = EL::cvt(q * ea);
                hk[(int)hh] = EL::cvt(k * ea);
                *reinterpret_cast<F *>(Kt + u * SK::VE + 4 * (int)hh) = EL::cvt(w * eb);
            });
            *reinterpret_cast<V8 *>(tg + CH * DK + row * DK + 8 * c) =
                __builtin_shufflevector(hqg[0], hqg[1], 0, 1, 2, 3, 4, 5, 6, 7);
            oq[(int)i] = __builtin_bit_cast(u32x4, __builtin_shufflevector(hq[0], hq[1], 0, 1, 2, 3, 4, 5, 6, 7));
            ok_[(int)i] = __builtin_bit_cast(u32x4, __builtin_shufflevector(hk[0], hk[1], 0, 1, 2, 3, 4, 5, 6, 7));
        });
        unroll<NPF>([&](auto m) {
            const int v = tid + NT * (int)m, vv = v < L::NL * DK ? v : 0;
            const int l = vv / DK, ch = vv % DK;
            int I = 0, J = l;
            while (J > I) { J -= I + 1; ++I; }
            opf[(int)m] = __expf(gam[16 * I * PG + ch] - gam[16 * J * PG + ch]);
        });
        float *gcb = reinterpret_cast<float *>(blk_base + CB::GOFF);
        for (int cc = tid; cc < DK; cc += NT) gcb[cc] = __expf(gam[(CH - 1) * PG + cc]);
        __syncthreads();                                       // flags set, decay table read
        int anyf = 0;
#pragma unroll
        for (int b = 0; b < NB; ++b) anyf |= flag[b];
        fast = anyf == 0;
        if (fast) {
            unroll<PER>([&](auto i) {
                const int u = (wave + (NT / 64) * (int)i) * 64 + lane;
                *reinterpret_cast<u32x4 *>(Qh + u * SK::VE) = oq[(int)i];
                *reinterpret_cast<u32x4 *>(Kh + u * SK::VE) = ok_[(int)i];
            });
            unroll<NPF>([&](auto m) {
                const int v = tid + NT * (int)m;
                if (v < L::NL * DK) PFs[v] = opf[(int)m];
            });
        } else {
            rk.store(Kst, tid);
            if constexpr (WR) rw.store(Wst, tid);
        }
    } else {
        rk.store(Kst, tid);
        if constexpr (!L::QREG) rq.store(Qst, tid);
        if constexpr (WR) rw.store(Wst, tid);
    }
    __syncthreads();
    if constexpr (GATE != 2) {
        // the state kernel's row factors (ChunkBlock)
        if (wave == 0 && lane < CH) {
            const float x = gam[lane], last = gam[CH - 1];
            const bool nrm = sizeof(E) == 2 && fz.qk_l2norm;
            const float fk = nrm ? rkf[lane] : 1.f, fq = nrm ? rqf[lane] : 1.f;
            const float gx = __expf(x);
            float *gblk = reinterpret_cast<float *>(blk_base + CB::GOFF);
            gblk[lane] = p.te_identity ? 0.f : gx * fk;          // GX = 0: X = V without the delta rule
            gblk[CH + lane] = p.scale * gx * fq;
            // zero past the end of the sequence: the state update scales those
            // rows of U~ (or V without the delta rule) by it, and the state
            // kernel leaves K and V rows there unzeroed
            gblk[2 * CH + lane] = lane < clen ? __expf(last - x) * fk : 0.f;
            if (lane < 4) gblk[3 * CH + lane] = lane == 0 ? __expf(last) : 0.f;
        }
    }

    // ---- K K^T (-> M) and Q K^T (-> A), lower tile pairs -----------------
    // Job (I, J) computes X = K_J Y_I^T for Y in {K, Q}; the C layout then
    // holds X[4g + jj][r] = <y_i, k_j> for i = 16I + r, j = 16J + 4g + jj, four
    // consecutive j of row i: exactly the fragment (I, J) of A / M.
    // job s of this wave -> tile (I, J); false past the wave's last job
    auto job_ij = [&](int s, int &I, int &J) __attribute__((always_inline)) {
        if constexpr (RB) {
            I = wave;
            J = s;
            return s <= wave;
        } else {
            const int job = wave + NW * s;
            I = 0;
            J = job;
            while (J > I) { J -= I + 1; ++I; }
            return job < NL;
        }
    };
    F bq_rb[RB && !L::LEAN ? NKB : 1], bk_rb[RB && !L::LEAN ? NKB : 1];  // row block I = wave, read once
    if constexpr (RB && !L::LEAN) {
#pragma unroll
        for (int kt = 0; kt < NKB; ++kt) {
            const int cc = 16 * kt + 4 * g4, irow = 16 * wave + r16;
            bq_rb[kt] = ld_frag<E>(Qst + SK::at(irow, cc));
            bk_rb[kt] = ld_frag<E>(Kst + SK::at(irow, cc));
        }
    }
    f32x4 res_q[JPW], res_k[JPW];
    // A and M tiles from the products' sums (C layout: row irow, columns 16 J + 4 g ..)
    auto job_tail = [&](int s, int I, int J, int irow, const f32x4 &accq, const f32x4 &acck)
        __attribute__((always_inline)) {
        f32x4 aq, mk;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int jt = 16 * J + 4 * g4 + jj;
            // computed for every lane and then selected: a lane-dependent branch
            // here becomes an exec-skip right after the MFMAs above
            float d = 1.f;
            if constexpr (GATE != 2) {
                const float e = __expf(gam[irow] - gam[jt]);
                d = (jt <= irow) ? e : 0.f;
            }
            aq[jj] = (jt <= irow) ? p.scale * accq[jj] * d : 0.f;
            mk[jj] = (jt < irow) ? bet[irow] * acck[jj] * d : 0.f;
        }
        if constexpr (GATE == 2) {
            // N itself (before diag(beta); with W, M = <k_i, w_j>), for the backward
            if (p.nout) {
                float *nb = p.nout + (slot * H + h) * CH * CH + irow * CH + 16 * J + 4 * g4;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) nb[jj] = 16 * J + 4 * g4 + jj < irow ? acck[jj] : 0.f;
            }
        }
        res_q[s] = aq;
        res_k[s] = mk;
    };
    if constexpr (L::FAST) {
        if (fast) {
            // gated operands from LDS: i side Qh, Kh; j side Kt * PF_IJ (pair l = job)
            const E *Kt = reinterpret_cast<const E *>(smem), *Qh = Kt + CH * DK, *Kh = Qh + CH * DK;
            const float *PFs = reinterpret_cast<const float *>(smem + 3 * CH * DK * (int)sizeof(E));
#pragma unroll
            for (int s = 0; s < JPW; ++s) {
                res_q[s] = res_k[s] = f32x4{0.f, 0.f, 0.f, 0.f};
                int I, J;
                if (!job_ij(s, I, J)) continue;
                const int l = wave + NW * s;
                const int jrow = 16 * J + r16, irow = 16 * I + r16;
                F a[NKB], bq[NKB], bk[NKB];
#pragma unroll
                for (int kt = 0; kt < NKB; ++kt) {
                    const int cc = 16 * kt + 4 * g4;
                    a[kt] = EL::cvt(EL::tof(ld_frag<E>(Kt + SK::at(jrow, cc))) * ld4(PFs + l * DK + cc));
                    bq[kt] = ld_frag<E>(Qh + SK::at(irow, cc));
                    bk[kt] = ld_frag<E>(Kh + SK::at(irow, cc));
                }
                f32x4 accq = {0.f, 0.f, 0.f, 0.f}, acck = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kt = 0; kt < NKB; kt += 2) {
                    accq = mfma_kb2(a[kt], bq[kt], a[kt + 1], bq[kt + 1], accq);
                    acck = mfma_kb2(a[kt], bk[kt], a[kt + 1], bk[kt + 1], acck);
                }
                job_tail(s, I, J, irow, accq, acck);
            }
        }
    }
    if constexpr (L::LEAN) {
        // row block I = wave against J = 0 .. I; A and M of each tile stored at once
        static_assert(RB, "one row block per wave");
        const int I = wave, irow = 16 * I + r16;
        if (irow >= clen) {
#pragma unroll
            for (int m = 0; m < NKB / 2; ++m) qfr[m] = V8{};
        }
        V8 bkr[NKB / 2];
#pragma unroll
        for (int m = 0; m < NKB / 2; ++m) bkr[m] = *reinterpret_cast<const V8 *>(Kst + SK::at(irow, 32 * m + 8 * g4));
        unroll<NB>([&](auto Jc) {
            constexpr int J = Jc;
            if (J > I) return;
            const int jrow = 16 * J + r16;
            f32x4 accq = {0.f, 0.f, 0.f, 0.f}, acck = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < NKB / 2; ++m) {
                const V8 a = *reinterpret_cast<const V8 *>(Kst + SK::at(jrow, 32 * m + 8 * g4));
                accq = mfma_pair(a, qfr[m], accq);
                acck = mfma_pair(a, bkr[m], acck);
            }
            job_tail(J, I, J, irow, accq, acck);
            st_frag<E>(blk + CH * CH + frag_pos<NB>(I, J, lane), EL::cvt(res_q[J]));
            if (p.use_delta) st4(Mf + mpos(I, J, r16, 4 * g4), res_k[J]);
        });
    }
#pragma unroll
    for (int s = 0; s < JPW; ++s) {
        if (fast || L::LEAN) break;
        res_q[s] = res_k[s] = f32x4{0.f, 0.f, 0.f, 0.f};
        int I, J;
        if (!job_ij(s, I, J)) continue;
        const int jrow = 16 * J + r16, irow = 16 * I + r16;
        F a[NKB], bq[NKB], bk[NKB];
        // QREG: Q row irow from global memory (a valid row, zeroed past the end),
        // rounded after the fused L2 norm as the staged rows are
        const E *qsrc = qg + (int64_t)(irow < clen ? irow : clen - 1) * sqk;
#pragma unroll
        for (int kt = 0; kt < NKB; ++kt) {
            const int cc = 16 * kt + 4 * g4;
            a[kt] = ld_frag<E>(Wst + SK::at(jrow, cc));           // the j side: the writing slot
            if constexpr (RB) {
                bq[kt] = bq_rb[kt];
                bk[kt] = bk_rb[kt];
            } else {
                if constexpr (L::QREG) bq[kt] = *reinterpret_cast<const F *>(qsrc + cc);
                else bq[kt] = ld_frag<E>(Qst + SK::at(irow, cc));
                bk[kt] = ld_frag<E>(Kst + SK::at(irow, cc));
            }
        }
        if constexpr (L::QREG) {
            const bool qn = sizeof(E) == 2 && fz.qk_l2norm;
            const float fq = qn ? rqf[irow] : 1.f;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                if (qn) bq[kt] = EL::cvt(EL::tof(bq[kt]) * fq);
                if (irow >= clen) bq[kt] = EL::cvt(f32x4{0.f, 0.f, 0.f, 0.f});
            }
        }
        bool pairwise = false;
        if constexpr (GATE == 2) {
            pairwise = (I == J) && flag[I];
            const int rr = 16 * I;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                const int cc = 16 * kt + 4 * g4;
                const f32x4 gr = ld4(gam + rr * PG + cc);
                const f32x4 ea = exp4(gr - ld4(gam + jrow * PG + cc));      // <= 1 off the diagonal
                const f32x4 eb = exp4(ld4(gam + irow * PG + cc) - gr);      // <= 1
                a[kt] = EL::cvt(EL::tof(a[kt]) * ea);
                bq[kt] = EL::cvt(EL::tof(bq[kt]) * eb);
                bk[kt] = EL::cvt(EL::tof(bk[kt]) * eb);
            }
        }
        f32x4 accq = {0.f, 0.f, 0.f, 0.f}, acck = {0.f, 0.f, 0.f, 0.f};
        if (!pairwise) {
#pragma unroll
            for (int kt = 0; kt < NKB; kt += 2) {
                accq = mfma_kb2(a[kt], bq[kt], a[kt + 1], bq[kt + 1], accq);
                acck = mfma_kb2(a[kt], bk[kt], a[kt + 1], bk[kt + 1], acck);
            }
        } else if constexpr (GATE == 2) {
            // exact pairwise products for a diagonal block with a large decay range
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int jt = 16 * J + 4 * g4 + jj;
                float sq = 0.f, sk = 0.f;
                if (jt <= irow) {
#pragma unroll 1
                    for (int cc = 0; cc < DK; cc += 4) {
                        const f32x4 e = exp4(ld4(gam + irow * PG + cc) - ld4(gam + jt * PG + cc));
                        const f32x4 kj = EL::tof(ld_frag<E>(Wst + SK::at(jt, cc))) * e;
                        f32x4 qv;
                        if constexpr (L::QREG) {                 // as bq above, before the gate
                            F qf = *reinterpret_cast<const F *>(qsrc + cc);
                            if (sizeof(E) == 2 && fz.qk_l2norm) qf = EL::cvt(EL::tof(qf) * rqf[irow]);
                            qv = irow < clen ? EL::tof(qf) : f32x4{0.f, 0.f, 0.f, 0.f};
                        } else {
                            qv = EL::tof(ld_frag<E>(Qst + SK::at(irow, cc)));
                        }
                        const f32x4 yq = qv * kj;
                        const f32x4 yk = EL::tof(ld_frag<E>(Kst + SK::at(irow, cc))) * kj;
                        sq += yq[0] + yq[1] + yq[2] + yq[3];
                        sk += yk[0] + yk[1] + yk[2] + yk[3];
                    }
                }
                accq[jj] = sq;
                acck[jj] = sk;
            }
        }
        job_tail(s, I, J, irow, accq, acck);
    }
    __syncthreads();                                           // K, Q reads done: M, T reuse the stage
#pragma unroll
    for (int s = 0; s < JPW; ++s) {
        int I, J;
        if (L::LEAN || !job_ij(s, I, J)) continue;
        if (!L::LEAN) st_frag<E>(blk + CH * CH + frag_pos<NB>(I, J, lane), EL::cvt(res_q[s]));
        if (p.use_delta) st4(Mf + mpos(I, J, r16, 4 * g4), res_k[s]);
    }
    // the upper tile (I, I + 1) shares a pair with diagonal tile (I, I) for even I: zeros
    if (wave < NB / 2) {
        const F zero = EL::cvt(f32x4{0.f, 0.f, 0.f, 0.f});
        st_frag<E>(blk + CH * CH + frag_pos<NB>(2 * wave, 2 * wave + 1, lane), zero);
        st_frag<E>(blk + frag_pos<NB>(2 * wave, 2 * wave + 1, lane), zero);
    }
    if (!p.use_delta) return;
    if (p.te_identity) {
        // TE = I: the delta form's blocks for U = V (no solve, beta unused)
        for (int tjob = wave; tjob < NL; tjob += NW) {
            int I = 0, kb = tjob;
            while (kb > I) { kb -= I + 1; ++I; }
            const int row = 16 * I + r16, c0 = 16 * kb + 4 * g4;
            f32x4 t;
#pragma unroll
            for (int e = 0; e < 4; ++e) t[e] = c0 + e == row ? 1.f : 0.f;
            st_frag<E>(blk + frag_pos<NB>(I, kb, lane), EL::cvt(t));
        }
        return;
    }
    __syncthreads();

    // ---- T = (I + M)^-1: 16x16 diagonal blocks by forward substitution ---
    if (wave == 0 && lane < 16 * NB) {
        const int b = lane >> 4, jc = lane & 15;
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float *mrow = Mf + mpos(b, b, i, 0);
            float acc = (i == jc) ? 1.f : 0.f;
#pragma unroll
            for (int m4 = 0; m4 < 16; m4 += 4) {
                if (m4 >= i) break;
                const f32x4 mv = ld4(mrow + m4);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (m4 + e < i) acc -= mv[e] * t[m4 + e];
            }
            t[i] = acc;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) Tf[mpos(b, b, i, jc)] = t[i];
    }
    __syncthreads();
    // off-diagonal blocks by distance: T_IJ = -T_II sum_{K=J}^{I-1} M_IK T_KJ
#pragma unroll
    for (int dist = 1; dist < NB; ++dist) {
        for (int J = wave; J < NB - dist; J += NW) {
            const int I = J + dist;
            f32x4 X = {0.f, 0.f, 0.f, 0.f};
            for (int K = J; K < I; ++K) {
                const float *tc = Tf + mpos(K, J, 4 * g4, r16);                   // column of T_KJ
                X = mfma_kb1(ld4(Mf + mpos(I, K, r16, 4 * g4)), f32x4{tc[0], tc[RS], tc[2 * RS], tc[3 * RS]}, X);
            }
            const f32x4 Y = mfma_kb1(ld4(Tf + mpos(I, I, r16, 4 * g4)), X, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int j = 0; j < 4; ++j) Tf[mpos(I, J, 4 * g4 + j, r16)] = -Y[j];
        }
        __syncthreads();
    }
    // ---- TE = T diag(beta), lower tiles, fragment order ---------------------
    for (int tjob = wave; tjob < NL; tjob += NW) {
        int I = 0, kb = tjob;
        while (kb > I) { kb -= I + 1; ++I; }
        const int row = 16 * I + r16, c0 = 16 * kb + 4 * g4;
        f32x4 t = ld4(Tf + mpos(I, kb, r16, 4 * g4)) * ld4(bet + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (c0 + e > row) t[e] = 0.f;
        st_frag<E>(blk + frag_pos<NB>(I, kb, lane), EL::cvt(t));
    }
}

// ===========================================================================
// chunk_state_kernel: the chunk recurrence and the outputs
// ===========================================================================
template <int DK, int CH, int NW, typename E, int GATE>
struct StateLayout {
    static constexpr int NT = 64 * NW, NB = CH / 16, NKB = DK / 16, DVT = 16 * NW;
    static constexpr int ES = sizeof(E);
    static constexpr int PC = CH + Elem<E>::pad;              // K^T pitch
    static constexpr int PV = DVT + Elem<E>::pad;             // output staging pitch
    // one double-buffer slot: K, Q (swizzled), V (swizzled), TE + A (fragment order), g (scalar gate)
    static constexpr int SLOT = (2 * CH * DK + CH * DVT + 2 * CH * CH) * ES + (GATE == 2 ? 0 : CH * 4);
    static constexpr int BYTES = 2 * SLOT + DK * PC * ES + CH * PV * ES + (GATE == 2 ? CH * DK * 4 : 4 * 4) +
                                 (2 * CH + (GATE == 2 ? DK : 4)) * 4;
    static constexpr bool FITS = BYTES <= 160 * 1024;
};

// One double-buffer slot of the state kernel.  The two slots are distinct LDS
// objects and every access names its slot at compile time, so the compiler
// can tell that reads of the current slot never alias the asynchronous copy
// into the other one (and does not make them wait for it).
template <int DK, int CH, int NW, typename E, int GATE>
struct StateSlot {
    E *K, *Q, *V, *B;
    float *g;
};

template <int V_> struct SlotTag { static constexpr int value = V_; };

// asynchronous copy of chunk c's operands (K, Q, V rows, TE + A blocks, scalar g)
template <int DK, int CH, int NW, typename E, int GATE>
__device__ __forceinline__ void state_issue(const StateSlot<DK, CH, NW, E, GATE> &sl, int c, int64_t bos, int64_t eos,
                                   int64_t cbase, int h, const E *kg, const E *qg, const E *vg, const E *blocks,
                                   const ChunkParams &p, int col0, int tid) {
    using L = StateLayout<DK, CH, NW, E, GATE>;
    const int H = p.H;
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * p.DV;
    const int64_t t0 = bos + (int64_t)c * CH;
    const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
    if constexpr (GATE != 2) {
        const int wave = tid >> 6, lane = tid & 63;
        if (wave == 0 && lane < CH && !(p.g && lane < clen)) sl.g[lane] = 0.f;
    }
    dma_rows<E, CH, DK, L::NT>(sl.K, kg + t0 * sqk, sqk, clen, DK, tid);
    dma_rows<E, CH, DK, L::NT>(sl.Q, qg + t0 * sqk, sqk, clen, DK, tid);
    dma_rows<E, CH, L::DVT, L::NT>(sl.V, vg + t0 * sv, sv, clen, p.DV - col0, tid);
    const char *bk = reinterpret_cast<const char *>(blocks) + ((cbase + c) * H + h) * ChunkBlock<E, CH, DK, GATE>::BYTES;
    dma_flat<E, 2 * CH * CH * L::ES / 16, L::NT>(sl.B, reinterpret_cast<const E *>(bk), tid);
    if constexpr (GATE != 2) {
        const int wave = tid >> 6, lane = tid & 63;
        if (wave == 0 && lane < CH && p.g && lane < clen) lds_dma4(p.g + (t0 + lane) * H + h, sl.g);
    }
}

template <int DK, int CH, int NW>
__device__ __forceinline__ void state_issue_g(float *gamv, int c, int64_t bos, int64_t eos, int h, const ChunkParams &p,
                                     int tid) {
    const int64_t t0 = bos + (int64_t)c * CH;
    const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
    dma_rows<float, CH, DK, 64 * NW, false>(gamv, p.g + (t0 * p.H + h) * DK, (int64_t)p.H * DK, clen, DK, tid);
}

template <int DK, int CH, int NW, typename E, int GATE, bool DELTA>
__global__ void __launch_bounds__(64 * NW) chunk_state_kernel(const ChunkParams p) {
    using L = StateLayout<DK, CH, NW, E, GATE>;
    static_assert(L::FITS, "LDS budget exceeded");
    using EL = Elem<E>;
    using F = typename EL::frag;
    using SK = Swz<E, DK>;
    using SV = Swz<E, L::DVT>;
    using Slot = StateSlot<DK, CH, NW, E, GATE>;
    constexpr int NT = L::NT, NB = L::NB, NKB = L::NKB, DVT = L::DVT;
    constexpr int PC = L::PC, PV = L::PV;

    __shared__ __attribute__((aligned(16))) E K0[CH * DK];
    __shared__ __attribute__((aligned(16))) E K1[CH * DK];
    __shared__ __attribute__((aligned(16))) E Q0[CH * DK];
    __shared__ __attribute__((aligned(16))) E Q1[CH * DK];
    __shared__ __attribute__((aligned(16))) E V0[CH * DVT];
    __shared__ __attribute__((aligned(16))) E V1[CH * DVT];
    __shared__ __attribute__((aligned(16))) E B0[2 * CH * CH];      // TE, then A
    __shared__ __attribute__((aligned(16))) E B1[2 * CH * CH];
    __shared__ __attribute__((aligned(16))) float g0[GATE == 2 ? 4 : CH];
    __shared__ __attribute__((aligned(16))) float g1[GATE == 2 ? 4 : CH];
    __shared__ __attribute__((aligned(16))) E KsT[DK * PC];
    __shared__ __attribute__((aligned(16))) E Os[CH * PV];
    __shared__ __attribute__((aligned(16))) float gamv[GATE == 2 ? CH * DK : 4];
    __shared__ __attribute__((aligned(16))) float Gs[CH];
    __shared__ __attribute__((aligned(16))) float Gend[CH];
    __shared__ __attribute__((aligned(16))) float Gc[GATE == 2 ? DK : 4];
    const Slot slot0{K0, Q0, V0, B0, g0}, slot1{K1, Q1, V1, B1, g1};

    // the wave index is uniform: readfirstlane makes every per-wave condition a scalar branch
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g4 = lane >> 4, r16 = lane & 15;
    const int H = p.H, DV = p.DV;

    // ---- work item: the dv tiles of one (sequence, head) share an XCD ------
    const int b = blockIdx.x;
    const int xcd = b & 7, y = b >> 3;
    const int tile = y % p.n_tiles;
    const int pos = (y / p.n_tiles) * 8 + xcd;
    if (pos >= p.geo.n_seqs * H) return;
    const int h = pos % H;
    const int spos = pos / H;
    const int seq = p.geo.order ? p.geo.order[spos] : spos;
    int64_t bos, eos;
    seq_bounds(p.geo, seq, bos, eos);
    const int64_t cbase = chunk_base(p.geo, seq);
    const int col0 = tile * DVT;
    const int wcol = 16 * wave;                                  // within the tile
    const bool wvalid = col0 + wcol < DV;                        // DV % 16 == 0
    const int64_t sv = (int64_t)H * DV;
    const E *kg = reinterpret_cast<const E *>(p.k) + (int64_t)h * DK;
    const E *qg = reinterpret_cast<const E *>(p.q) + (int64_t)h * DK;
    const E *vg = reinterpret_cast<const E *>(p.v) + (int64_t)h * DV + col0;
    E *og = reinterpret_cast<E *>(p.o) + (int64_t)h * DV + col0;
    const E *blocks = reinterpret_cast<const E *>(p.blocks);

    // ---- entry state (C layout: S[kt][j] = S[16kt + 4g + j][col0 + wcol + r16]) --
    f32x4 S[NKB];
    const int64_t sbase = ((int64_t)seq * H + h) * DK * DV + col0 + wcol + r16;
#pragma unroll
    for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            S[kt][j] = (p.h0 && wvalid) ? p.h0[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] : 0.f;

    const int64_t len = eos - bos;
    const int nchunks = (int)((len + CH - 1) / CH);

    // outputs of a finished chunk: staged rows -> global, 16-byte stores
    constexpr int VE = 16 / L::ES;
    auto flush = [&](int64_t t0, int clen) {
        for (int vi = tid; vi < CH * (DVT / VE); vi += NT) {
            const int row = vi / (DVT / VE), col = (vi % (DVT / VE)) * VE;
            if (row < clen && col0 + col < DV) {
                const uint2 *s2 = reinterpret_cast<const uint2 *>(Os + row * PV + col);
                const uint2 lo = s2[0], hi = s2[1];
                *reinterpret_cast<Vec16 *>(og + (t0 + row) * sv + col) = Vec16{{lo.x, lo.y, hi.x, hi.y}};
            }
        }
    };

    // one chunk, with its operands in slot SL (known at compile time)
    auto step = [&](auto tag, int c) {
        constexpr int SL = decltype(tag)::value;
        const Slot &cur = SL ? slot1 : slot0;
        const Slot &nxt = SL ? slot0 : slot1;
        const int64_t t0 = bos + (int64_t)c * CH;
        const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
        E *Kst = cur.K;
        E *Qst = cur.Q;
        const E *Vst = cur.V;
        const E *TEs = cur.B;
        const E *Aqs = cur.B + CH * CH;

        dma_wait();
        lds_barrier();                                        // chunk c landed; chunk c-1 fully consumed
        if (c + 1 < nchunks)                                  // into the slot chunk c-1 used
            state_issue<DK, CH, NW, E, GATE>(nxt, c + 1, bos, eos, cbase, h, kg, qg, vg, blocks, p, col0, tid);
        if (c > 0) flush(t0 - CH, CH);                        // every chunk but the last is full

        // ---- gates and the transposed keys --------------------------------
        if constexpr (GATE == 2) {
            // per-channel inclusive scan: NP parts of SEG tokens per channel
            static_assert(NT % DK == 0, "one or more whole threads per channel");
            constexpr int NP = NT / DK;
            constexpr int SEG = CH / NP;
            {
                const int cc = tid % DK, part = tid / DK;
                float acc = 0.f;
                for (int t = part * SEG; t < (part + 1) * SEG; ++t) {
                    acc += gamv[t * DK + cc];
                    gamv[t * DK + cc] = acc;
                }
            }
            if constexpr (NP > 1) {
                lds_barrier();
                const int cc = tid % DK, part = tid / DK;
                float off = 0.f;
                for (int q2 = 0; q2 < part; ++q2) off += gamv[((q2 + 1) * SEG - 1) * DK + cc];
                lds_barrier();
                if (part > 0)
                    for (int t = part * SEG; t < (part + 1) * SEG; ++t) gamv[t * DK + cc] += off;
            }
            lds_barrier();
            for (int cc = tid; cc < DK; cc += NT) Gc[cc] = __expf(gamv[(CH - 1) * DK + cc]);
            // KsT = (K * Gend)^T, K <- K * G, Q <- scale * Q * G (each element owned by one item)
            for (int it = tid; it < DK * (CH / 4); it += NT) {
                const int cc = it % DK, t = (it / DK) * 4;
                const float last = gamv[(CH - 1) * DK + cc];
                const f32x4 gm = {gamv[(t + 0) * DK + cc], gamv[(t + 1) * DK + cc], gamv[(t + 2) * DK + cc],
                                  gamv[(t + 3) * DK + cc]};
                const f32x4 G = exp4(gm), Ge = exp4(last - gm);
                f32x4 kx;
#pragma unroll
                for (int e = 0; e < 4; ++e) kx[e] = EL::to_f(Kst[SK::at(t + e, cc)]);
                st_frag<E>(KsT + cc * PC + t, EL::cvt(kx * Ge));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    Kst[SK::at(t + e, cc)] = EL::from_f(kx[e] * G[e]);
                    Qst[SK::at(t + e, cc)] = EL::from_f(EL::to_f(Qst[SK::at(t + e, cc)]) * G[e] * p.scale);
                }
            }
        } else {
            if (wave == 0) {
                float x = cur.g[lane < CH ? lane : CH - 1];
                if (lane >= CH) x = 0.f;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const float yv = __shfl_up(x, o);
                    if (lane >= o) x += yv;
                }
                const float last = __shfl(x, CH - 1);
                if (lane < CH) {
                    Gs[lane] = __expf(x);
                    Gend[lane] = __expf(last - x);
                }
                if (lane == 0) Gc[0] = __expf(last);
            }
            for (int it = tid; it < DK * (CH / 4); it += NT) {
                const int cc = it % DK, t = (it / DK) * 4;
                F x = {Kst[SK::at(t, cc)], Kst[SK::at(t + 1, cc)], Kst[SK::at(t + 2, cc)], Kst[SK::at(t + 3, cc)]};
                st_frag<E>(KsT + cc * PC + t, x);
            }
        }
        lds_barrier();
        if constexpr (GATE == 2) {
            if (c + 1 < nchunks) state_issue_g<DK, CH, NW>(gamv, c + 1, bos, eos, h, p, tid);   // buffer is free
        }

        // ---- this wave's 16 state columns ---------------------------------
        if (wvalid) {
            F Sb[NKB];
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) Sb[kt] = EL::cvt(S[kt]);
            f32x4 U[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I)
#pragma unroll
                for (int j = 0; j < 4; ++j) U[I][j] = EL::to_f(Vst[SV::at(16 * I + 4 * g4 + j, wcol + r16)]);
            if constexpr (DELTA) {
                // X = V - (K*G) S  (independent accumulation chains per token block) ;  U~ = TE X
                f32x4 P[NB];
#pragma unroll
                for (int I = 0; I < NB; ++I) P[I] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kt = 0; kt < NKB; kt += 2) {
                    F a0[NB], a1[NB];
#pragma unroll
                    for (int I = 0; I < NB; ++I) {
                        a0[I] = ld_frag<E>(Kst + SK::at(16 * I + r16, 16 * kt + 4 * g4));
                        a1[I] = ld_frag<E>(Kst + SK::at(16 * I + r16, 16 * kt + 16 + 4 * g4));
                    }
#pragma unroll
                    for (int I = 0; I < NB; ++I) P[I] = mfma_kb2(a0[I], Sb[kt], a1[I], Sb[kt + 1], P[I]);
                }
                F Xb[NB];
#pragma unroll
                for (int I = 0; I < NB; ++I) {
                    if constexpr (GATE != 2) P[I] *= ld4(Gs + 16 * I + 4 * g4);
                    Xb[I] = EL::cvt(U[I] - P[I]);
                }
#pragma unroll
                for (int I = 0; I < NB; ++I)
                    U[I] = contract(f32x4{0.f, 0.f, 0.f, 0.f}, I + 1,
                        [&](int kb) { return ld_frag<E>(TEs + frag_pos<NB>(I, kb, lane)); },
                        [&](int kb) { return Xb[kb]; });
            }
            F Ub[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) Ub[I] = EL::cvt(U[I]);
            // o = scale (Q*G) S + A U~   -> staging rows
            f32x4 O[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) O[I] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < NKB; kt += 2) {
                F a0[NB], a1[NB];
#pragma unroll
                for (int I = 0; I < NB; ++I) {
                    a0[I] = ld_frag<E>(Qst + SK::at(16 * I + r16, 16 * kt + 4 * g4));
                    a1[I] = ld_frag<E>(Qst + SK::at(16 * I + r16, 16 * kt + 16 + 4 * g4));
                }
#pragma unroll
                for (int I = 0; I < NB; ++I) O[I] = mfma_kb2(a0[I], Sb[kt], a1[I], Sb[kt + 1], O[I]);
            }
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                if constexpr (GATE != 2) O[I] *= ld4(Gs + 16 * I + 4 * g4) * p.scale;
                O[I] = contract(O[I], I + 1,
                    [&](int kb) { return ld_frag<E>(Aqs + frag_pos<NB>(I, kb, lane)); },
                    [&](int kb) { return Ub[kb]; });
                E *orow = Os + (16 * I + 4 * g4) * PV + wcol + r16;
#pragma unroll
                for (int j = 0; j < 4; ++j) orow[j * PV] = EL::from_f(O[I][j]);
            }
            // S <- Gc (.) S + (K*Gend)^T U~   (independent chains per key block)
            F Wb[NB];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                if constexpr (GATE != 2) Wb[I] = EL::cvt(U[I] * ld4(Gend + 16 * I + 4 * g4));
                else Wb[I] = Ub[I];
            }
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt) {
                if constexpr (GATE == 2) S[kt] *= ld4(Gc + 16 * kt + 4 * g4);
                else S[kt] *= Gc[0];
            }
#pragma unroll
            for (int kb = 0; kb < NB; kb += 2) {
                F a0[NKB], a1[NKB];
#pragma unroll
                for (int kt = 0; kt < NKB; ++kt) {
                    a0[kt] = ld_frag<E>(KsT + (16 * kt + r16) * PC + 16 * kb + 4 * g4);
                    a1[kt] = ld_frag<E>(KsT + (16 * kt + r16) * PC + 16 * kb + 16 + 4 * g4);
                }
#pragma unroll
                for (int kt = 0; kt < NKB; ++kt) S[kt] = mfma_kb2(a0[kt], Wb[kb], a1[kt], Wb[kb + 1], S[kt]);
            }
        }
        (void)clen;
    };

    if (nchunks > 0) {
        state_issue<DK, CH, NW, E, GATE>(slot0, 0, bos, eos, cbase, h, kg, qg, vg, blocks, p, col0, tid);
        if constexpr (GATE == 2) state_issue_g<DK, CH, NW>(gamv, 0, bos, eos, h, p, tid);
    }
    for (int c = 0; c < nchunks; c += 2) {
        step(SlotTag<0>{}, c);
        if (c + 1 < nchunks) step(SlotTag<1>{}, c + 1);
    }
    lds_barrier();
    if (nchunks > 0) {
        const int64_t tl = bos + (int64_t)(nchunks - 1) * CH;
        flush(tl, (int)(eos - tl));
    }

    if (p.ht && wvalid) {
#pragma unroll
        for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
            for (int j = 0; j < 4; ++j) p.ht[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] = S[kt][j];
    }
}

// ===========================================================================
// helpers of the 16-bit state kernel (LDS transpose reads, producer copies)
// ===========================================================================
// Values the compiler must treat as unknown where they are produced.  Address
// arithmetic derived from them is redone next to each use instead of being
// hoisted out of the chunk loop, which would pin one register per fragment
// address (and per slot) for the whole kernel.
__device__ __forceinline__ int opaque_v(int x) { asm volatile("" : "+v"(x)); return x; }
__device__ __forceinline__ int opaque_s(int x) { asm volatile("" : "+s"(x)); return x; }
// the value is computed at this point in program order
template <typename T> __device__ __forceinline__ void pin_v(const T &x) { asm volatile("" ::"v"(x)); }

// LDS layout of the 16-bit state kernel's K rows.  Rows are padded by 32 bytes and every
// fragment address is a per-lane base plus a compile-time offset.  Measured on
// gfx950 (8 waves on one CU): the 16-byte fragment reads of 16 rows and the
// transpose reads of 4 rows x 4 lanes both run conflict-free at a 288-byte
// row pitch (3.9 cycles per wave instruction) and take twice as long at 272
// bytes; the LDS serves 256 bytes per clock to conflict-free 16-byte reads.  K and Q
// rows hold their columns in paired order: the 16-byte unit 4 q + g of a row
// holds columns 32 q + 4 g .. + 3 and 32 q + 16 + 4 g .. + 3, the eight
// elements lane group g contributes to one 16x16x32 MFMA over k-blocks
// (2 q, 2 q + 1) -- one 16-byte read per MFMA operand.
template <int DK>
struct KQRows {
    static constexpr int PITCH = DK + 16;                              // elements
    // element offset of column c (a multiple of 4) within a row
    __host__ __device__ static constexpr int col(int c) { return (c / 32) * 32 + ((c % 16) / 4) * 8 + ((c % 32) / 16) * 4; }
};

// Copies by the producer waves: plain 16-byte global loads into registers
// (every load of a chunk in flight at once), then LDS stores.  Measured on
// MI355X with all CUs streaming data not yet cached, this path moves several
// times more bytes per CU than global_load_lds, whose throughput from HBM is
// far lower than from L2.  Rows [0, CH) x columns [0, NCOL) of a token-major
// matrix; rows >= valid_rows and columns >= valid_cols hold some other finite
// element of the tile (see below).
// PAIRED: the K/Q column order above; else the source order.  PITCH: LDS row
// pitch in elements.
//
// Every load is issued unconditionally, from unit 0 (always inside the tile)
// where the unit itself is out of range: loads under a per-lane branch made
// the wait-count insertion put a full vmcnt(0) wait in front of each following
// load, which serialised them.  Such a unit is not zeroed either: a row past
// the end of a sequence has beta = 0 and zero k, q in chunk_prep, so its
// columns of TE and A are exactly zero, and its decay Gend (which scales its
// row of U~, or of V without the delta rule, in the state update) is written
// as zero; per-channel gates zero its K*Gend row instead.  Any finite value
// in its K, Q or V row then contributes nothing, and its output row is not
// stored.  Columns past dv belong to 16-column strips no compute wave uses.
// The registers are a vector type: a 16-byte struct copied under a condition
// becomes a memcpy through a stack slot, which the alloca promotion pass then
// moves to LDS or scratch.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// lane l receives x from lane l ^ 2 (DPP quad_perm [2, 3, 0, 1]; register only)
__device__ __forceinline__ uint32_t from_lane_xor2(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false);
}

// PAIRED (the K/Q layout): loads are the plain contiguous ones (lane l: unit l
// of its row group); lanes l and l ^ 2 hold units u and u ^ 2 of one
// 32-column group, swap halves through DPP, and each writes one whole paired
// unit: 4 q + 2 a from units 4 q + a, 4 q + a + 2 (the lower halves) or
// 4 q + 2 a + 1 (the upper halves).
//
// Which units a lane moves, and where they sit in global memory relative to
// the chunk's first row and in LDS, is the same for every chunk: Plan holds
// it, computed once; a chunk then costs one 64-bit add per load.
template <typename E, int CH, int NCOL, int NPT, bool PAIRED, int PITCH>
struct RowCopy {
    static constexpr int VE = 16 / (int)sizeof(E), UPR = NCOL / VE, UNITS = CH * UPR;
    static constexpr int PER = (UNITS + NPT - 1) / NPT;
    static_assert(PER <= 32, "one bit per unit");
    static_assert(!PAIRED || (UPR % 4 == 0 && NPT % 64 == 0), "quads of lanes hold whole 32-column groups");
    struct Plan {
        int64_t goff[PER];                                   // elements from the chunk's first row
        int row[PER];
        int loff[PER];                                       // LDS elements
        uint32_t exists = 0, cols = 0, lo = 0;               // unit < UNITS; columns < valid_cols; PAIRED half
    };
    __device__ static __forceinline__ Plan plan(int64_t stride, int valid_cols, int pt) {
        Plan pl;
        unroll<PER>([&](auto i) {
            const int u0 = pt + NPT * i;
            const bool ex = UNITS % NPT == 0 || u0 < UNITS;
            const int u = ex ? u0 : 0, row = u / UPR, cu = u % UPR, a = cu & 3;
            pl.goff[i] = (int64_t)row * stride + cu * VE;
            pl.row[i] = row;
            pl.loff[i] = row * PITCH + (PAIRED ? 32 * (cu >> 2) + (a < 2 ? 16 * a : 16 * (a - 2) + 8) : cu * VE);
            pl.exists |= (uint32_t)ex << (int)i;
            pl.cols |= (uint32_t)(cu * VE < valid_cols) << (int)i;
            pl.lo |= (uint32_t)(a < 2) << (int)i;
        });
        return pl;
    }
    u32x4 r[PER];
    __device__ __forceinline__ void load(const E *src, const Plan &pl, int valid_rows) {
        unroll<PER>([&](auto i) {
            const bool ok = (pl.exists & pl.cols) >> (int)i & 1u && pl.row[i] < valid_rows;
            r[i] = *reinterpret_cast<const u32x4 *>(src + (ok ? pl.goff[i] : 0));
        });
    }
    __device__ __forceinline__ void store(E *lds, const Plan &pl) const {
        unroll<PER>([&](auto i) {
            const u32x4 x = r[i];
            u32x4 d = x;
            if constexpr (PAIRED) {
                u32x4 o;                                       // unit cu ^ 2, from lane ^ 2
                unroll<4>([&](auto k) { o[(int)k] = from_lane_xor2(x[(int)k]); });
                d = (pl.lo >> (int)i) & 1u ? u32x4{x[0], x[1], o[0], o[1]} : u32x4{o[2], o[3], x[2], x[3]};
            }
            if ((pl.exists >> (int)i) & 1u) *reinterpret_cast<u32x4 *>(lds + pl.loff[i]) = d;
        });
    }
};

// Contiguous 16-byte units (the chunk_prep block), loaded as above.
template <int UNITS, int NPT>
struct FlatCopy {
    static constexpr int PER = (UNITS + NPT - 1) / NPT;
    u32x4 r[PER];
    __device__ __forceinline__ void load(const void *src, int pt) {
        unroll<PER>([&](auto i) {
            const int u = pt + NPT * i;
            r[i] = reinterpret_cast<const u32x4 *>(src)[UNITS % NPT == 0 || u < UNITS ? u : 0];
        });
    }
    __device__ __forceinline__ void store(void *lds, int pt) const {
        unroll<PER>([&](auto i) {
            const int u = pt + NPT * i;
            if (UNITS % NPT == 0 || u < UNITS) reinterpret_cast<u32x4 *>(lds)[u] = r[i];
        });
    }
};

// The TE block's tile pairs that can be nonzero (frag_pair_pos order, pair (I, q)
// with 2 q <= I; the chain never reads the others): with four row blocks, six of
// the eight pairs, 384 of the 512 16-byte units.  Unit n of the copy is unit n % 64
// of the (n / 64)-th such pair.  A lane past the last unit reads through a buffer
// resource at an offset outside it (no memory request, zeros) and stores nothing,
// so every wave runs the same instructions without a branch around a load.
template <int NB, int NPT>
struct TECopy {
    static constexpr int NPAIRS = NB * (NB / 2);                         // all tile pairs of the block
    static constexpr int LIVE = NB == 4 ? 384 : 64 * NPAIRS;             // units of the pairs with 2 q <= I
    static constexpr int PER = (LIVE + NPT - 1) / NPT;
    static_assert(NB == 4 || NB == 2, "four or two row blocks");
    u32x4 r[PER];
    // byte offset of unit n within the block (n < LIVE)
    __device__ static __forceinline__ uint32_t unit_off(int n) {
        if constexpr (NB == 4) {
            const int j = n >> 6;                                          // 0..5 -> pairs 0, 2, 4, 5, 6, 7
            const int pair = j == 0 ? 0 : (j == 1 ? 2 : j + 2);
            return (uint32_t)((pair * 64 + (n & 63)) * 16);
        } else {
            return (uint32_t)(n * 16);
        }
    }
    __device__ __forceinline__ void load(const void *src, int pt) {
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(src, (uint32_t)(NPAIRS * 64 * 16));
        unroll<PER>([&](auto i) {
            const int n = pt + NPT * i;
            const uint32_t off = (LIVE % NPT == 0 || n < LIVE) ? unit_off(n) : 0x80000000u;
            r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0));
        });
    }
    __device__ __forceinline__ void store(void *lds, int pt) const {
        unroll<PER>([&](auto i) {
            const int n = pt + NPT * i;
            if (LIVE % NPT == 0 || n < LIVE)
                *reinterpret_cast<u32x4 *>(reinterpret_cast<char *>(lds) + unit_off(n)) = r[i];
        });
    }
};

// Q rows (VEC: the scaled Q*G tile) for the output waves.  The global units are
// the K copy's (its Plan: sixteen consecutive lanes read one whole row, so each
// load instruction covers whole cache lines; loading the MFMA operand straight
// from global memory spread every instruction over sixteen rows, 64 bytes
// each, which measured 4 % slower on the whole state kernel).  In LDS the rows
// are unpadded and 16-byte unit u of row r sits at unit u ^ qswz(r): the output
// waves' operand reads (one unit of each of sixteen rows per lane group) then
// hit distinct banks.
template <int DK>
__device__ __forceinline__ int qswz(int row) {
    if constexpr (DK == 128) return row & 15;
    else return (row ^ (row >> 3)) & 7;                      // DK = 64: two rows per 256 bytes
}
template <typename E, int CH, int DK, int NPT>
struct QCopy {
    static_assert(DK == 128 || DK == 64, "key dims 64 and 128");
    static constexpr int UPR = DK / 8, UNITS = CH * UPR;
    static constexpr int PER = (UNITS + NPT - 1) / NPT;
    u32x4 r[PER];
    template <typename Plan>
    __device__ __forceinline__ void load(const E *src, const Plan &pl, int valid_rows) {
        unroll<PER>([&](auto i) {
            const bool ok = (pl.exists & pl.cols) >> (int)i & 1u && pl.row[i] < valid_rows;
            r[i] = *reinterpret_cast<const u32x4 *>(src + (ok ? pl.goff[i] : 0));
        });
    }
    __device__ __forceinline__ void store(E *lds, int pt) const {
        unroll<PER>([&](auto i) {
            const int u = pt + NPT * i;
            if (UNITS % NPT == 0 || u < UNITS) {
                const int row = u / UPR, cu = u % UPR;
                *reinterpret_cast<u32x4 *>(lds + row * DK + 8 * (cu ^ qswz<DK>(row))) = r[i];
            }
        });
    }
};

template <typename E>
__device__ __forceinline__ typename Elem<E>::frag2 ld_pair(const E *p) {
    return *reinterpret_cast<const typename Elem<E>::frag2 *>(p);
}
// two transpose reads (k-blocks 2 q and 2 q + 1) as one MFMA operand
template <typename E>
__device__ __forceinline__ typename Elem<E>::frag2 ld_tr_pair(const E *p0, const E *p1) {
    const typename Elem<E>::frag a = ld_tr<E>(p0), b = ld_tr<E>(p1);
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// ===========================================================================
// chunk_pipe_kernel: the chunk recurrence for 16-bit elements, with the
// outputs computed one chunk behind by waves of their own
// ===========================================================================
// The recurrence S_c -> S_c+1 is the only sequential part of the prefill; the
// outputs o_c = GO Q_c S_c + A_c U~_c hang off it.  One workgroup per
// (sequence, head, 16 NW-column dv tile) splits its waves by role:
//   chain waves   0 .. NW - 1     wave w owns columns col0 + 16 w .. + 15 of the
//                                  state as fp32 C-layout accumulators for the whole
//                                  sequence and runs only the recurrence:
//                                  P = K S, X = V - GX P, U~ = TE X,
//                                  S <- Gc S + (GE K)^T U~  (per-channel gate: K*G,
//                                  K*Gend tiles and Gc per key channel).  For each
//                                  chunk it leaves S_c (element type) and U~_c in LDS.
//   output waves  NW .. NW + NO - 1  compute chunk c's O^T = S_c^T (GO Q)^T + U~_c^T A^T
//                                  for all NW column strips, 1 / NO of the token
//                                  blocks each, while the chain runs chunk c + 1.  A comes
//                                  from global memory straight into registers, issued
//                                  two hand-overs before it is used; Q (or scale Q*G)
//                                  from LDS (four producer waves) or, like A, from
//                                  global memory (two).
//   producers     NW + NO ..       copy chunk c + 1's K (K*G and K*Gend), V, TE and gate
//                                  factors into the idle half of the double buffer,
//                                  and chunk c's Q into its own double buffer.
// The chain waves thus issue 38 of the 60 MFMAs per chunk and column strip, and
// the output products run on the other SIMDs (waves w and NW + w sit on
// different SIMDs of the CU whenever NW <= 2).
//
// Barriers: b = 0 .. n (n chunks).  Barrier b hands operand slot b & 1 (chunk b)
// to the chain waves and hand-over buffer (b - 1) & 1 (chunk b - 1) to the output
// waves; every role passes all n + 1 of them.  Writes to a hand-over buffer
// (chain, during step c) and its reads (output, during step c + 1) are separated
// by barrier c + 1, and the next write to it (step c + 2) by barrier c + 2.  The
// same holds for Q slot c & 1: written during step c, read during step c + 1.
//
// Hand-over layout per chain wave and buffer:
//   SH: the state in the element type, one row of DK + 8 elements per state
//       column (natural key order), so the output wave reads eight consecutive
//       keys per lane and its Q operand is eight consecutive keys of a q row;
//   UH: U~ in the MFMA A-operand order the chain wave holds it (lane-to-lane).
// HS: the output waves also store each chunk's entry state to p.hs
// ([chunk slot, H] checkpoints in ckpt_pos order), for the chunked backward.
// OUT false (with HS): only those states -- no outputs, so no U~ hand-over,
// no Q copy and no A, Q loads or products in the output waves; the backward's
// entry-state walk.
template <int DK, int CH, int NW, int NP, typename E, bool VEC, bool DELTA, bool HS = false, bool OUT = true,
          int NO = 2>
__global__ void __launch_bounds__(64 * (NW + NO + NP))
__attribute__((amdgpu_waves_per_eu(1, (NW + NO + NP + 3) / 4)))
chunk_pipe_kernel(const ChunkParams p) {
    static_assert(sizeof(E) == 2, "transpose reads take 16-bit elements");
    using EL = Elem<E>;
    using F2 = typename EL::frag2;
    typedef E E4 __attribute__((ext_vector_type(4)));
    using CB = ChunkBlock<E, CH, DK, VEC ? 2 : 1>;
    using KQ = KQRows<DK>;
    constexpr int NB = CH / 16, NKB = DK / 16, DVT = 16 * NW, NPT = 64 * NP;
    constexpr int PK = KQ::PITCH, PV = (VEC && NW == 4) ? DVT + 8 : DVT + 16;
    constexpr int SP = DK + 8;                                   // hand-over state row pitch (elements)
    constexpr int TEB = CH * CH * (int)sizeof(E);                // bytes of TE in a slot
    constexpr int FB = CB::FLOATS * 4;                           // bytes of the gate factors
    static_assert(NB % 2 == 0 && NKB % 2 == 0, "k-blocks are consumed in pairs");
    static_assert(TEB % 16 == 0 && FB % 16 == 0, "slots are copied in 16-byte units");
    // Q through LDS (copied by the producers) when there are four producer waves;
    // with two, their registers are full and the output waves load the Q operand
    // straight from global memory (the whole-row loads and an LDS transpose in
    // the output waves measured no faster there)
    constexpr bool QL = NP >= 4 && OUT;
    static_assert(OUT || HS, "a walk without outputs stores the entry states");

    __shared__ __attribute__((aligned(16))) E K0[CH * PK];
    __shared__ __attribute__((aligned(16))) E K1[CH * PK];
    __shared__ __attribute__((aligned(16))) E KE0[VEC ? CH * PK : 8];
    __shared__ __attribute__((aligned(16))) E KE1[VEC ? CH * PK : 8];
    __shared__ __attribute__((aligned(16))) E V0[CH * PV];
    __shared__ __attribute__((aligned(16))) E V1[CH * PV];
    __shared__ __attribute__((aligned(16))) char B0[TEB + FB];
    __shared__ __attribute__((aligned(16))) char B1[TEB + FB];
    __shared__ __attribute__((aligned(16))) E SH[2 * NW * 16 * SP];
    __shared__ __attribute__((aligned(16))) E UH[2 * NW * (NB / 2) * 64 * 8];
    __shared__ __attribute__((aligned(16))) E QS[QL ? 2 * CH * DK : 8];  // Q (VEC: Q*G), slot c & 1: chunk c

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int H = p.H, DV = p.DV;

    // ---- work item: the dv tiles of one (sequence, head) share an XCD ------
    const int b = blockIdx.x;
    const int xcd = b & 7, y = b >> 3;
    const int tile = y % p.n_tiles;
    const int pos = (y / p.n_tiles) * 8 + xcd;
    if (pos >= p.geo.n_seqs * H) return;
    const int h = pos % H;
    const int spos = pos / H;
    const int seq = p.geo.order ? p.geo.order[spos] : spos;
    int64_t bos, eos;
    seq_bounds(p.geo, seq, bos, eos);
    const int64_t cbase = chunk_base(p.geo, seq);
    const int col0 = tile * DVT;
    const int64_t sqk = (int64_t)H * DK, sv = (int64_t)H * DV;
    const E *kg = reinterpret_cast<const E *>(p.k) + (int64_t)h * DK;
    const E *qg = reinterpret_cast<const E *>(p.q) + (int64_t)h * DK;
    const E *vg = reinterpret_cast<const E *>(p.v) + (int64_t)h * DV + col0;
    const char *blocks = reinterpret_cast<const char *>(p.blocks);
    const int64_t len = eos - bos;
    const int nchunks = (int)((len + CH - 1) / CH);

    // ======================= producers ======================================
    if (wave >= NW + NO) {
        using CK = RowCopy<E, CH, DK, NPT, !VEC, PK>;            // K rows (VEC: K*G and K*Gend tiles)
        using CV = RowCopy<E, CH, DVT, NPT, false, PV>;
        struct Staged {
            CK k, e;
            CV v;
            TECopy<NB, NPT> t;
            FlatCopy<FB / 16, NPT> f;
        };
        using CQ = QCopy<E, CH, DK, NPT>;
        struct Plans {
            typename CK::Plan k;
            typename CV::Plan v;
        };
        // a chunk index past the end loads the last chunk again (every address
        // stays inside the tensors); store(st, c) writes slot c & 1
        auto load = [&](Staged &st, const Plans &pl, int c, int pt) __attribute__((always_inline)) {
            c = c < nchunks ? c : nchunks - 1;
            const int64_t t0 = bos + (int64_t)c * CH;
            const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
            const char *bk = blocks + ((cbase + c) * H + h) * (int64_t)CB::BYTES;
            st.t.load(bk, pt);
            st.f.load(bk + CB::GOFF, pt);
            if constexpr (VEC) {
                const E *tiles = reinterpret_cast<const E *>(bk) + CB::TEA;
                st.k.load(tiles, pl.k, CH);
                st.v.load(vg + t0 * sv, pl.v, clen);
                st.e.load(tiles + 2 * CH * DK, pl.k, CH);
            } else {
                st.k.load(kg + t0 * sqk, pl.k, clen);
                st.v.load(vg + t0 * sv, pl.v, clen);
            }
        };
        auto store = [&](const Staged &st, const Plans &pl, int c, int z, int pt) __attribute__((always_inline)) {
            const bool odd = c & 1;
            st.t.store((odd ? B1 : B0) + z, pt);
            st.f.store((odd ? B1 : B0) + z + TEB, pt);
            st.k.store((odd ? K1 : K0) + z, pl.k);
            st.v.store((odd ? V1 : V0) + z, pl.v);
            if constexpr (VEC) st.e.store((odd ? KE1 : KE0) + z, pl.k);
        };
        // Q of chunk c goes to Q slot c & 1 between barriers c and c + 1 (the output
        // waves read it one step after the chain reads chunk c's K).  Each Q load is
        // issued before the next K loads, so that the wait for it leaves those in
        // flight.
        auto load_q = [&](CQ &qc, const Plans &pl, int c) __attribute__((always_inline)) {
            c = c < nchunks ? c : nchunks - 1;
            if constexpr (VEC) {
                const char *bq = blocks + ((cbase + c) * H + h) * (int64_t)CB::BYTES;
                qc.load(reinterpret_cast<const E *>(bq) + CB::TEA + CH * DK, pl.k, CH);
            } else {
                const int64_t tq = bos + (int64_t)c * CH;
                qc.load(qg + tq * sqk, pl.k, (int)(eos - tq < CH ? eos - tq : CH));
            }
        };
        if (nchunks > 0) {
            const int pt = tid - 64 * (NW + NO);
            const Plans pl{CK::plan(VEC ? DK : sqk, DK, pt), CV::plan(sv, DV - col0, pt)};
            Staged s0, s1;
            // per-channel gate: Q*G of the even chunks in qa, of the odd ones in qb,
            // each loaded two steps ahead (kda_prefill state kernel 194.4 -> 190.9 us);
            // the scalar gate loads Q one step ahead into qa alone (two sets measured
            // 93.4 -> 94.5 us at gdn_340m)
            constexpr bool Q2 = VEC;
            CQ qa, qb;
            CQ &qo = Q2 ? qb : qa;
            load(s0, pl, 0, pt);
            store(s0, pl, 0, 0, pt);
            if constexpr (QL) {
                load_q(qa, pl, 0);
                if constexpr (Q2) load_q(qb, pl, 1);
            }
            load(s1, pl, 1, pt);
            load(s0, pl, 2, pt);
            int c = 0;
            for (; c + 1 < nchunks; c += 2) {
                int z = opaque_s(0);
                lds_barrier();                                // barrier c: chunk c in place, chunk c-1 consumed
                store(s1, pl, c + 1, z, pt);                  // into the slot chunk c-1 used
                if constexpr (QL) {
                    qa.store(QS + z, pt);                     // Q of chunk c (even)
                    load_q(qa, pl, Q2 ? c + 2 : c + 1);
                }
                load(s1, pl, c + 3, pt);
                z = opaque_s(0);
                lds_barrier();                                // barrier c + 1
                store(s0, pl, c + 2, z, pt);
                if constexpr (QL) {
                    qo.store(QS + CH * DK + z, pt);           // Q of chunk c + 1 (odd)
                    load_q(qo, pl, Q2 ? c + 3 : c + 2);
                }
                load(s0, pl, c + 4, pt);
            }
            if (c < nchunks) {                                // n odd: c = n - 1, even
                const int z = opaque_s(0);
                lds_barrier();                                // barrier n - 1
                if constexpr (QL) qa.store(QS + z, pt);       // the last chunk's Q
            }
            lds_barrier();                                    // barrier n: the last chunk's outputs
            __builtin_amdgcn_s_waitcnt(0);                    // no load left in flight at exit
        }
        return;
    }

    // ======================= chain waves ====================================
    if (wave < NW) {
        const int wcol = 16 * wave;
        const bool wvalid = col0 + wcol < DV;                  // DV % 16 == 0
        // entry state (C layout: S[kt][j] = S[16kt + 4g + j][col0 + wcol + r])
        f32x4 S[NKB];
        {
            const int g4 = lane >> 4, r16 = lane & 15;
            const int64_t sbase = ((int64_t)seq * H + h) * DK * DV + col0 + wcol + r16;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    S[kt][j] = (p.h0 && wvalid) ? p.h0[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] : 0.f;
        }
        for (int c = 0; c < nchunks; ++c) {
            const int z = opaque_s(0);
            lds_barrier();                                    // barrier c
            if (!wvalid) continue;
            const int ln = opaque_v(lane);
            const int g4 = ln >> 4, r16 = ln & 15;
            const bool odd = c & 1;
            // per-lane bases; every fragment below is base + a compile-time offset
            const E *Krow = (odd ? K1 : K0) + z + r16 * PK + 8 * g4;                 // row r, unit g
            const E *Ktr = (VEC ? (odd ? KE1 : KE0) : (odd ? K1 : K0)) + z + (4 * g4 + (r16 >> 2)) * PK + 8 * (r16 & 3);
            const E *Vtr = (odd ? V1 : V0) + z + (4 * g4 + (r16 >> 2)) * PV + wcol + 4 * (r16 & 3);
            const char *Bst = (odd ? B1 : B0) + z;
            const E *TEs = reinterpret_cast<const E *>(Bst) + 8 * ln;
            // scalar gate: GX, GO, GE, Gc (ChunkBlock); VEC: Gc per key channel
            const float *gs = reinterpret_cast<const float *>(Bst + TEB), *ge = gs + 2 * CH;
            E *sh = SH + ((odd ? NW : 0) + wave) * 16 * SP + z + r16 * SP + 4 * g4;
            E *uh = UH + ((odd ? NW : 0) + wave) * (NB / 2) * 512 + z + 8 * ln;

            // Operands that do not depend on the state are read first, in one
            // batch (the scheduler would otherwise issue each next to its use,
            // one LDS round trip apiece on the critical path): the gate factors,
            // TE, the V rows.
            f32x4 gx[NB], gev[NB], gcv[VEC ? NKB : 1];
            float gc = 0.f;
            F2 te[NB][NB / 2];
            typename EL::frag vf[NB];
            if constexpr (VEC) {
                unroll<NKB>([&](auto kt) { gcv[kt] = ld4(gs + 16 * kt + 4 * g4); });     // Gc per key channel
            } else {
                unroll<NB>([&](auto I) {
                    gx[I] = ld4(gs + 16 * I + 4 * g4);
                    gev[I] = ld4(ge + 16 * I + 4 * g4);
                });
                gc = gs[3 * CH];
            }
            if constexpr (DELTA)
                unroll<NB>([&](auto I) {
                    unroll<NB / 2>([&](auto q) {
                        if (2 * q <= I) te[I][q] = ld_pair<E>(TEs + frag_pair_pos<NB>(I, q, 0));
                    });
                });
            // V rows in C layout: V[16 I + 4 g + j][wcol + r]
            unroll<NB>([&](auto I) { vf[I] = ld_tr<E>(Vtr + 16 * I * PV); });
            __builtin_amdgcn_sched_barrier(0);

            F2 Sb[NKB / 2];
#pragma unroll
            for (int q = 0; q < NKB / 2; ++q) {
                Sb[q] = EL::cvt2(S[2 * q], S[2 * q + 1]);
                // rows 32 q + 4 g .. + 3 and 32 q + 16 + 4 g .. + 3 of column r
                *reinterpret_cast<E4 *>(sh + 32 * q) = __builtin_shufflevector(Sb[q], Sb[q], 0, 1, 2, 3);
                *reinterpret_cast<E4 *>(sh + 32 * q + 16) = __builtin_shufflevector(Sb[q], Sb[q], 4, 5, 6, 7);
            }
            f32x4 U[NB];
            if constexpr (DELTA) {
                // P = K S (C layout), NB independent accumulation chains
                f32x4 P[NB];
#pragma unroll
                for (int I = 0; I < NB; ++I) P[I] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q = 0; q < NKB / 2; ++q)
#pragma unroll
                    for (int I = 0; I < NB; ++I) P[I] = mfma_pair(ld_pair<E>(Krow + 16 * I * PK + 32 * q), Sb[q], P[I]);
                // X = V - GX P ;  U~ = TE X
                F2 Xb[NB / 2];
#pragma unroll
                for (int q = 0; q < NB / 2; ++q) {
                    if constexpr (VEC) Xb[q] = EL::cvt2(EL::tof(vf[2 * q]) - P[2 * q], EL::tof(vf[2 * q + 1]) - P[2 * q + 1]);
                    else Xb[q] = EL::cvt2(EL::tof(vf[2 * q]) - P[2 * q] * gx[2 * q],
                                          EL::tof(vf[2 * q + 1]) - P[2 * q + 1] * gx[2 * q + 1]);
                }
#pragma unroll
                for (int I = 0; I < NB; ++I) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int q = 0; 2 * q <= I; ++q) acc = mfma_pair(te[I][q], Xb[q], acc);
                    U[I] = acc;
                }
            } else {
                unroll<NB>([&](auto I) { U[I] = EL::tof(vf[I]); });
            }
            F2 Wb[NB / 2];
#pragma unroll
            for (int q = 0; q < NB / 2; ++q) {
                const F2 ub = EL::cvt2(U[2 * q], U[2 * q + 1]);
                if constexpr (OUT) *reinterpret_cast<F2 *>(uh + 512 * q) = ub;
                if constexpr (VEC) Wb[q] = ub;                     // Gend is in the K*Gend tile
                else Wb[q] = EL::cvt2(U[2 * q] * gev[2 * q], U[2 * q + 1] * gev[2 * q + 1]);
            }
            // S <- Gc S + (K*Gend)^T U~
            if constexpr (VEC) {
#pragma unroll
                for (int kt = 0; kt < NKB; ++kt) S[kt] *= gcv[kt];
            } else {
#pragma unroll
                for (int kt = 0; kt < NKB; ++kt) S[kt] *= gc;
            }
#pragma unroll
            for (int q = 0; q < NB / 2; ++q)
#pragma unroll
                for (int kt = 0; kt < NKB; ++kt)
                    S[kt] = mfma_pair(ld_tr_pair<E>(Ktr + 32 * q * PK + KQ::col(16 * kt),
                                                    Ktr + (32 * q + 16) * PK + KQ::col(16 * kt)), Wb[q], S[kt]);
        }
        if (nchunks > 0) lds_barrier();                       // barrier n
        if (p.ht && wvalid) {
            const int g4 = lane >> 4, r16 = lane & 15;
            const int64_t sbase = ((int64_t)seq * H + h) * DK * DV + col0 + wcol + r16;
#pragma unroll
            for (int kt = 0; kt < NKB; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) p.ht[sbase + (int64_t)(16 * kt + 4 * g4 + j) * DV] = S[kt][j];
        }
        return;
    }

    // ======================= output waves ===================================
    // Output wave o covers token blocks rb(o, 0), rb(o, 1) ({0, 3} and {1, 2} at
    // CH = 64, the same A tile pairs each) of every column strip of the tile.
    // Three register sets of operands: chunk c + 2's loads are issued when chunk
    // c's outputs start, two hand-overs before they are used.
    static_assert(NO == 2 || NO == NB, "two output waves, or one per token block");
    constexpr int NR = NB / NO;                                // token blocks per output wave
    const int o = wave - NW;
    auto rb = [&](int i) { return NO == NB ? o : (i == 0 ? o : NB - 1 - o); };
    if (nchunks == 0) return;
    const int g4 = lane >> 4, r16 = lane & 15;
    struct Ops {
        F2 q[QL ? 1 : NR][NKB / 2];                            // !QL: Q rows 16 rb(i) + r, keys 32 k + 8 g .. + 7
        F2 a[NR][NB / 2];                                      // A tile pairs (rb(i), k), 2 k <= rb(i)
        float go[NR];
    };
    auto oload = [&](Ops &op, int c) __attribute__((always_inline)) {
        if constexpr (!OUT) return;
        c = c < nchunks ? c : nchunks - 1;                     // past the end: the last chunk again
        const int64_t t0 = bos + (int64_t)c * CH;
        const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
        const char *bk = blocks + ((cbase + c) * H + h) * (int64_t)CB::BYTES;
        const E *Ab = reinterpret_cast<const E *>(bk) + CH * CH;
        const float *gof = reinterpret_cast<const float *>(bk + CB::GOFF) + CH;
        unroll<NR>([&](auto i) {
            const int I = rb(i), row = 16 * I + r16;
            if constexpr (!QL) {
                // rows past the end of the sequence read its last row (not stored)
                const E *qrow;
                if constexpr (VEC) qrow = reinterpret_cast<const E *>(bk) + CB::TEA + CH * DK + row * DK;
                else qrow = qg + (t0 + (row < clen ? row : clen - 1)) * sqk;
                unroll<NKB / 2>([&](auto k) { op.q[i][k] = *reinterpret_cast<const F2 *>(qrow + 32 * k + 8 * g4); });
            }
            unroll<NB / 2>([&](auto k) {
                if (2 * k <= I) op.a[i][k] = *reinterpret_cast<const F2 *>(Ab + frag_pair_pos<NB>(I, k, lane));
            });
            if constexpr (!VEC) op.go[i] = gof[row];
        });
    };
    // O^T = S^T (GO Q)^T + U~^T A^T for chunk c: lane (g, r) ends with columns
    // 16 s + 4 g .. + 3 of token 16 I + r.  The hand-over of every strip is read
    // first; the NW x NR accumulators then advance together (independent MFMA
    // chains, interleaved).
    auto oproducts = [&](const Ops &op, int c, int z) __attribute__((always_inline)) {
        const int64_t t0 = bos + (int64_t)c * CH;
        const int clen = (int)(eos - t0 < CH ? eos - t0 : CH);
        const bool odd = c & 1;
        F2 Sn[NW][NKB / 2], Ub[NW][NB / 2], Qv[NR][NKB / 2];
        // Q rows 16 rb(i) + r, keys 32 k + 8 g .. + 7 (rows past the end of the
        // sequence hold other rows' values; their outputs are not stored)
        unroll<NR>([&](auto i) {
            if constexpr (QL) {
                const int row = 16 * rb(i) + r16;
                const E *qs = QS + (odd ? CH * DK : 0) + z + row * DK;
                unroll<NKB / 2>([&](auto k) {
                    Qv[i][k] = *reinterpret_cast<const F2 *>(qs + 8 * ((4 * k + g4) ^ qswz<DK>(row)));
                });
            } else {
                unroll<NKB / 2>([&](auto k) { Qv[i][k] = op.q[i][k]; });
            }
        });
        unroll<NW>([&](auto s) {
            const E *sh = SH + ((odd ? NW : 0) + s) * 16 * SP + z + r16 * SP;
            const E *uh = UH + ((odd ? NW : 0) + s) * (NB / 2) * 512 + z + 8 * lane;
            unroll<NKB / 2>([&](auto k) { Sn[s][k] = *reinterpret_cast<const F2 *>(sh + 32 * k + 8 * g4); });
            unroll<NB / 2>([&](auto k) { Ub[s][k] = *reinterpret_cast<const F2 *>(uh + 512 * k); });
        });
        f32x4 ot[NW][NR];
        unroll<NW>([&](auto s) { unroll<NR>([&](auto i) { ot[s][i] = f32x4{0.f, 0.f, 0.f, 0.f}; }); });
        unroll<NKB / 2>([&](auto k) {
            unroll<NW>([&](auto s) { unroll<NR>([&](auto i) { ot[s][i] = mfma_pair(Sn[s][k], Qv[i][k], ot[s][i]); }); });
        });
        if constexpr (!VEC)                                    // VEC: scale and G are in Q*G
            unroll<NW>([&](auto s) { unroll<NR>([&](auto i) { ot[s][i] *= op.go[i]; }); });
        unroll<NB / 2>([&](auto k) {
            unroll<NW>([&](auto s) {
                unroll<NR>([&](auto i) {
                    if (2 * k <= rb(i)) ot[s][i] = mfma_pair(Ub[s][k], op.a[i][k], ot[s][i]);
                });
            });
        });
        // the chunk's o rows as one buffer: rows past the sequence's end fall
        // outside it and their stores are dropped, with no lane-dependent branch
        const __amdgpu_buffer_rsrc_t ors =
            buffer_rsrc(reinterpret_cast<E *>(p.o) + t0 * sv + (int64_t)h * DV + col0, (uint32_t)(clen * sv * sizeof(E)));
        if constexpr (NW % 2 == 0) {
            // strips 2 m and 2 m + 1 leave as 16-byte units: lanes l and l ^ 16 trade
            // halves (v_permlane16_swap), after which lane (g, r) holds eight consecutive
            // columns of row r -- strip 2 m + (g & 1), columns 8 (g >> 1) .. + 7 -- and
            // each store writes 64 contiguous bytes of 16 rows (8-byte stores wrote
            // 32-byte pieces, a quarter of a cache line, which cost HBM write
            // efficiency).  A lane whose columns lie past dv gets an offset outside
            // the buffer, so its store is dropped without a branch.
            unroll<NR>([&](auto i) {
                const int I = rb(i);
                unroll<NW / 2>([&](auto m) {
                    const u32x2 x = __builtin_bit_cast(u32x2, EL::cvt(ot[2 * m][i]));
                    const u32x2 y = __builtin_bit_cast(u32x2, EL::cvt(ot[2 * m + 1][i]));
                    const auto a = __builtin_amdgcn_permlane16_swap(x[0], y[0], false, false);
                    const auto b = __builtin_amdgcn_permlane16_swap(x[1], y[1], false, false);
                    const int col = 32 * m + 16 * (g4 & 1) + 8 * (g4 >> 1);
                    const uint32_t off = col0 + col < DV ? (uint32_t)(((16 * I + r16) * sv + col) * sizeof(E))
                                                         : 0x80000000u;
                    __builtin_amdgcn_raw_buffer_store_b128(u32x4{a[0], b[0], a[1], b[1]}, ors, (int)off, 0, 0);
                });
            });
        }
        if constexpr (NW % 2 != 0)
            unroll<NW>([&](auto s) {
                if (col0 + 16 * s >= DV) return;
                unroll<NR>([&](auto i) {
                    const int I = rb(i);
                    buffer_store_8b(EL::cvt(ot[s][i]), ors,
                                    (uint32_t)(((16 * I + r16) * sv + 16 * s + 4 * g4) * sizeof(E)));
                });
            });
    };
    auto ocompute = [&](const Ops &op, int c, int z) __attribute__((always_inline)) {
        const bool odd = c & 1;
        if constexpr (OUT) oproducts(op, c, z);
        if constexpr (HS)
            unroll<NW>([&](auto s) {
                if (col0 + 16 * s >= DV) return;
                // the checkpoint's fragment order: lane (g, r) holds rows 16 kt + 4 g .. + 3
                // of column 16 cb + r.  Output wave o stores key blocks o, o + NO, ..
                const E *sh = SH + ((odd ? NW : 0) + s) * 16 * SP + z + r16 * SP;
                E *hs = reinterpret_cast<E *>(p.hs) + ((cbase + c) * H + h) * (int64_t)DK * DV;
                const int cb = (col0 >> 4) + s;
                unroll<NKB / NO>([&](auto k) {
                    const int kt = NO * k + o;
                    *reinterpret_cast<E4 *>(hs + ckpt_pos<DK>(cb, kt, lane)) =
                        *reinterpret_cast<const E4 *>(sh + 16 * kt + 4 * g4);
                });
            });
    };
    Ops o0, o1, o2;
    oload(o0, 0);
    oload(o1, 1);
    lds_barrier();                                            // barrier 0
    int c = 0;
    for (; c + 2 < nchunks; c += 3) {
        int z;
        oload(o2, c + 2);
        z = opaque_s(0);
        lds_barrier();                                        // barrier c + 1: chunk c's hand-over
        ocompute(o0, c, z);
        oload(o0, c + 3);
        z = opaque_s(0);
        lds_barrier();
        ocompute(o1, c + 1, z);
        oload(o1, c + 4);
        z = opaque_s(0);
        lds_barrier();
        ocompute(o2, c + 2, z);
    }
    if (c < nchunks) {
        const int z = opaque_s(0);
        lds_barrier();
        ocompute(o0, c, z);
    }
    if (c + 1 < nchunks) {
        const int z = opaque_s(0);
        lds_barrier();
        ocompute(o1, c + 1, z);
    }
    __builtin_amdgcn_s_waitcnt(0);                            // no load left in flight at exit
}

// ===========================================================================
// launch
// ===========================================================================
// The delta rule is a template parameter of the state kernel: a run-time
// branch around the TE product put a control-flow join right after its last
// MFMA, and for chunk_state_kernel<64, 64, 2, bf16/f16, 2> hipcc (AMD clang 22)
// then emitted reads of that MFMA's accumulators without the required wait
// states (wrong outputs in token block 3).  Without the join there is no
// such read.
template <int DK, int CH, typename E, bool VEC, bool DELTA, bool HS, bool OUT = true>
static void launch_pipe(const ChunkParams &p, int nw, int64_t state_blocks, hipStream_t stream) {
    const dim3 grid((unsigned)state_blocks);
    if constexpr (!VEC) {
        if (nw == 4) {
            // 64-column tiles (packed batches with many (sequence, head) pairs): four
            // producers (Q through LDS) and one output wave per token block, 12 waves
            // at 164 VGPRs; gdn_varlen 604.5 -> 585.4 us against two producers and two
            // output waves (four producers with two output waves: 590.0 us)
            constexpr int NO = CH / 16;                       // one output wave per token block
            hipLaunchKernelGGL((chunk_pipe_kernel<DK, CH, 4, 4, E, VEC, DELTA, HS, OUT, NO>), grid,
                               dim3(64 * (8 + NO)), 0, stream, p);
            return;
        }
    }
    if (nw == 2)
        hipLaunchKernelGGL((chunk_pipe_kernel<DK, CH, 2, 4, E, VEC, DELTA, HS, OUT>), grid, dim3(64 * 8), 0, stream, p);
    else
        hipLaunchKernelGGL((chunk_pipe_kernel<DK, CH, 1, 4, E, VEC, DELTA, HS, OUT>), grid, dim3(64 * 7), 0, stream, p);
}

template <int DK, int CH, typename E, int GATE, bool DELTA>
static void launch_state(const ChunkParams &p, int nw, int64_t state_blocks, hipStream_t stream) {
    if constexpr (sizeof(E) == 2) {
        // 16-bit elements: the pipelined kernel (chain, output and producer waves)
        constexpr bool VEC = GATE == 2;
        if constexpr (DELTA) {
            if (p.hs) {                                       // a training forward: entry states saved
                if (p.states_only)                            // the backward's walk: no outputs
                    launch_pipe<DK, CH, E, VEC, true, true, false>(p, nw, state_blocks, stream);
                else
                    launch_pipe<DK, CH, E, VEC, true, true>(p, nw, state_blocks, stream);
                return;
            }
        }
        launch_pipe<DK, CH, E, VEC, DELTA, false>(p, nw, state_blocks, stream);
        return;
    } else {
    if constexpr (StateLayout<DK, CH, 4, E, GATE>::FITS) {
        if (nw == 4) {
            hipLaunchKernelGGL((chunk_state_kernel<DK, CH, 4, E, GATE, DELTA>), dim3((unsigned)state_blocks),
                               dim3(256), 0, stream, p);
            return;
        }
    }
    hipLaunchKernelGGL((chunk_state_kernel<DK, CH, 2, E, GATE, DELTA>), dim3((unsigned)state_blocks), dim3(128), 0,
                       stream, p);
    }
}

template <int DK, int CH, typename E, int GATE>
static hipError_t launch_chunk(const ChunkParams &p, int nw, int phases, hipStream_t stream) {
    const int64_t prep_blocks = (int64_t)p.n_chunk_slots * p.H;
    if ((phases & CHUNK_PREP) && prep_blocks > 0) {
        bool done = false;
        if constexpr (GATE == 2 && sizeof(E) == 2) {
            if (p.w) {
                hipLaunchKernelGGL((chunk_prep_kernel<DK, CH, E, GATE, true>), dim3((unsigned)prep_blocks), dim3(256),
                                   0, stream, p);
                done = true;
            }
        }
        if (!done) {
            if (p.w) return hipErrorInvalidValue;             // the API admits w only on the 16-bit per-channel path
            hipLaunchKernelGGL((chunk_prep_kernel<DK, CH, E, GATE>), dim3((unsigned)prep_blocks), dim3(256), 0,
                               stream, p);
        }
    }
    const int64_t units = (int64_t)p.geo.n_seqs * p.H;
    const int64_t state_blocks = (units + 7) / 8 * 8 * p.n_tiles;
    if ((phases & CHUNK_STATE) && state_blocks > 0) {
        if (p.use_delta) launch_state<DK, CH, E, GATE, true>(p, nw, state_blocks, stream);
        else launch_state<DK, CH, E, GATE, false>(p, nw, state_blocks, stream);
    }
    return hipGetLastError();
}

template <int DK, int CH, typename E, int GATE>
static int state_waves(int64_t units, int dv, int cus) {
    if constexpr (sizeof(E) == 2) {
        // the widest tile (16 nw columns) that still gives every CU a workgroup;
        // 64-column tiles only with the scalar gate (the per-channel tiles overflow LDS)
        if (GATE != 2 && units * ((dv + 63) / 64) >= cus) return 4;
        return units * ((dv + 31) / 32) >= cus ? 2 : 1;
    } else {
        // fp32: 64-column tiles once the (sequence, head) pairs fill the chip and the tile fits LDS
        if (!StateLayout<DK, CH, 4, E, GATE>::FITS) return 2;
        return units * ((dv + 63) / 64) >= cus ? 4 : 2;
    }
}

int64_t chunk_blocks_bytes(int dtype, int chunk, int64_t chunk_slots, int64_t H, int64_t dk, int gate_vector) {
    const int64_t es = dtype == 0 ? 4 : 2;
    const bool vec = gate_vector && dtype != 0;                            // ChunkBlock<E, chunk, dk, gate>::BYTES
    const int64_t per = 2 * chunk * chunk * es + (vec ? 3 * chunk * dk * es + dk * 4 : (3 * chunk + 4) * 4);
    return chunk_slots * H * per;
}

template <int DK, int CH, typename E, int GATE>
static hipError_t run_chunk(ChunkParams p, int phases, hipStream_t stream) {
    const int nw = state_waves<DK, CH, E, GATE>((int64_t)p.geo.n_seqs * p.H, p.DV, device_cu_count());
    p.n_tiles = (p.DV + 16 * nw - 1) / (16 * nw);
    return launch_chunk<DK, CH, E, GATE>(p, nw, phases, stream);
}

hipError_t chunk_fwd(int dtype, int dk, int chunk, int gate_vector, ChunkParams p, int32_t *table, int phases,
                     hipStream_t stream) {
    if (p.geo.n_seqs == 0) return hipSuccess;                  // nothing to do (and no table to read)
    if (p.geo.cu) {
        if (phases & CHUNK_PREP) {
            hipError_t e = varlen_prepare(p.geo.cu, p.geo.n_seqs, p.geo.n_tokens, chunk, table, stream);
            if (e != hipSuccess) return e;
        }
        p.geo.chunk_offs = table + 2 * p.geo.n_seqs;
        p.geo.order = table + 3 * p.geo.n_seqs + 1;
    }
#define VGDR_GATES(DK_, CH_, E_)                                                           \
    return gate_vector ? run_chunk<DK_, CH_, E_, 2>(p, phases, stream) : run_chunk<DK_, CH_, E_, 1>(p, phases, stream);
    if (dtype == 1) {
        if (dk == 64) { if (chunk == 32) { VGDR_GATES(64, 32, __bf16) } VGDR_GATES(64, 64, __bf16) }
        if (chunk == 32) { VGDR_GATES(128, 32, __bf16) } VGDR_GATES(128, 64, __bf16)
    }
    if (dtype == 2) {
        if (dk == 64) { if (chunk == 32) { VGDR_GATES(64, 32, _Float16) } VGDR_GATES(64, 64, _Float16) }
        if (chunk == 32) { VGDR_GATES(128, 32, _Float16) } VGDR_GATES(128, 64, _Float16)
    }
    // fp32 runs 32-token chunks (the double-buffered fp32 tiles of 64 tokens overflow LDS)
    if (dk == 64) { VGDR_GATES(64, 32, float) }
    VGDR_GATES(128, 32, float)
#undef VGDR_GATES
}

}  // namespace vgdr

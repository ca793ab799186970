// Backward of the token recurrence for every scan form the chunked backward
// does not take: the per-channel (KDA) gate, the explicit write vector w (the
// asymmetric delta rule) and the plain, no-delta recurrence.  The scalar gate
// and no gate run here too.
//
// Per head, with a_t = exp(g_t) (scalar or per key row) and the write vector
// x_t = beta_t k_t, or w_t, or (no delta rule) k_t (linear_attention.py:161-195):
//     S~_t = Diag(a_t) S_{t-1}
//     u_t  = v_t - S~_t^T k_t            (u_t = v_t without the delta rule)
//     S_t  = S~_t + x_t u_t^T
//     o_t  = scale S_t^T q_t
// and, walking back with dS the gradient of S_t (dht at the end):
//     dS   += scale q_t do_t^T
//     dq_t  = scale S_t do_t
//     dx_t  = dS u_t                      (no delta: this is dk_t)
//     du_t  = dS^T x_t   = dv_t
//     dS~   = dS - k_t du_t^T             (no delta: dS~ = dS)
//     dk_t  = -S~_t du_t                  (+ beta_t dx_t for x = beta k; dbeta_t = k_t . dx_t)
//     dg_t  = rowsum(dS~ o S~_t)          (summed over rows for a scalar gate)
//     dS    = Diag(a_t) dS~               (dh0 at the start)
//
// The state's columns evolve independently, so one workgroup owns one
// (sequence, head, tile of TW = 4 * waves columns) and each of its waves four
// of those columns over all DK rows (lane l: rows l*RPL .. l*RPL + RPL - 1),
// with no barrier in either walk: the only reductions, over the key rows
// (S~^T k and dS^T x), stay inside the wave (DPP row rotations and row
// broadcasts, then one readlane).
//
// scan_walks_kernel runs the two sequential walks side by side: forward,
// storing S at the entry of every block of CT tokens and u_t of every token;
// and back, storing dS at every block's exit and writing dv (the dS recurrence
// needs no state).  scan_grad_kernel then takes every block at once: it
// recomputes the block's states from the entry checkpoint and u (two FMAs per
// element, no reduction), walks the block back from its exit gradient, and
// adds the sums over the columns (dq, dk, dx, dg) into LDS, leaving one fp32
// partial per (tile, token, head, row); scan_bwd_finish_kernel adds the tiles
// and applies the write vector's chain rule.
#include "gdr_common.hpp"
#include "gdr_chunk_layout.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

constexpr int SB_CT = 8;   // tokens per checkpoint block

int64_t scan_bwd_ckpt_slots(int64_t n_tokens, int64_t n_seqs) { return n_tokens / SB_CT + n_seqs + 1; }

namespace {

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_src(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK,
                                                                 0xf, false));
}

// the sum of x over the wave's 64 lanes, returned to every lane: rotations
// within each 16-lane row leave the row's sum in all its lanes, the two row
// broadcasts carry rows 0..2 into row 3, and lane 63's value is read out
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_src<0x128>(x);          // row_ror:8
    x += dpp_src<0x124>(x);          // row_ror:4
    x += dpp_src<0x122>(x);          // row_ror:2
    x += dpp_src<0x121>(x);          // row_ror:1
    x += dpp_src<0x142, 0xa>(x);     // row_bcast:15 into rows 1 and 3
    x += dpp_src<0x143, 0xc>(x);     // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// four wave sums at once, stage by stage, so that the four DPP chains overlap
__device__ __forceinline__ void wave_sum4(float (&x)[4]) {
    unroll<4>([&](auto j) __attribute__((always_inline)) { x[j] += dpp_src<0x128>(x[j]); });
    unroll<4>([&](auto j) __attribute__((always_inline)) { x[j] += dpp_src<0x124>(x[j]); });
    unroll<4>([&](auto j) __attribute__((always_inline)) { x[j] += dpp_src<0x122>(x[j]); });
    unroll<4>([&](auto j) __attribute__((always_inline)) { x[j] += dpp_src<0x121>(x[j]); });
    unroll<4>([&](auto j) __attribute__((always_inline)) { x[j] += dpp_src<0x142, 0xa>(x[j]); });
    unroll<4>([&](auto j) __attribute__((always_inline)) { x[j] += dpp_src<0x143, 0xc>(x[j]); });
    unroll<4>([&](auto j) __attribute__((always_inline)) {
        x[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x[j]), 63));
    });
}

template <typename E, int N>
__device__ __forceinline__ void load_f(const E *__restrict__ p, float (&x)[N]) {
    unroll<N>([&](auto i) __attribute__((always_inline)) { x[i] = Elem<E>::to_f(p[i]); });
}

// a lane's RPL consecutive row values as one load: RPL = 2 packs two 16-bit
// elements into one register
template <typename T, int RPL> struct RowVec { typedef T V __attribute__((ext_vector_type(RPL))); };
template <typename T> struct RowVec<T, 1> { typedef T V; };
template <typename T, int RPL>
__device__ __forceinline__ typename RowVec<T, RPL>::V ld_row(const T *p) {
    return *reinterpret_cast<const typename RowVec<T, RPL>::V *>(p);
}
template <typename T, int RPL>
__device__ __forceinline__ float row_el(typename RowVec<T, RPL>::V x, int r) {
    if constexpr (RPL == 1) return Elem<T>::to_f(x); else return Elem<T>::to_f(x[r]);
}
__device__ __forceinline__ float lane_val(float x, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

// One block of CT tokens as a lane holds it before use, fetched a block ahead
// and left raw until then (a conversion would wait for the load).  Row data
// per lane; the wave-uniform per-token values spread over lanes and read back
// with readlane: lane 4i + j holds u (or v) of token i, column j, lane
// 32 + 4i + j its do; lane i its scalar gate and beta.
template <int RPL, typename E>
struct Blk {
    typename RowVec<E, RPL>::V q[SB_CT], k[SB_CT], w[SB_CT];
    typename RowVec<float, RPL>::V g[SB_CT];
    float s0[RPL][4];      // the block's entry state (backward)
    float uf;              // u (delta rule, backward)
    E vr, dr;              // v, do
    float gs, bs;          // scalar gate, beta
};

template <int RPL, typename E>
__device__ __forceinline__ void load_blk(const ScanBwdParams &p, Blk<RPL, E> &b, int64_t bos, int64_t L, int64_t t0,
                                         int h, int row0, int lane, int col0, bool bwd, const float *ck,
                                         bool need_uv = true) {
    constexpr int DK = RPL * 64;
    const int H = p.H, DV = p.DV;
    auto th = [&](int64_t i) {
        const int64_t t = t0 + i;
        return (bos + (t < L ? t : L - 1)) * H + h;
    };
    const E *qp = reinterpret_cast<const E *>(p.q), *kp = reinterpret_cast<const E *>(p.k);
    unroll<SB_CT>([&](auto i) __attribute__((always_inline)) {
        const int64_t o = th(i) * DK + row0;
        b.k[i] = ld_row<E, RPL>(kp + o);
        if (bwd) b.q[i] = ld_row<E, RPL>(qp + o);
        if (p.mode == 1) b.w[i] = ld_row<E, RPL>(reinterpret_cast<const E *>(p.w) + o);
        if (p.gate == 2) b.g[i] = ld_row<float, RPL>(p.g + o);
    });
    const int li = lane & 31;
    const int64_t tu = th(li >> 2) * DV + col0 + (li & 3);
    // (the reverse walk reads neither: its dS recurrence needs q, k, the write
    // vector, the gate and do, and u is being written by the forward walk of
    // the same launch)
    if (need_uv) {
        if (bwd && p.mode != 2) b.uf = p.u[tu];
        else b.vr = reinterpret_cast<const E *>(p.v)[tu];
    }
    if (bwd) b.dr = reinterpret_cast<const E *>(p.dout)[tu];
    const int64_t ts = th(lane & (SB_CT - 1));
    if (p.gate == 1) b.gs = p.g[ts];
    if (p.mode == 0) b.bs = p.beta[ts];
    if (ck) {
        unroll<RPL>([&](auto r) __attribute__((always_inline)) {
            const f32x4 x = ld4(ck + r * 4);
            unroll<4>([&](auto j) __attribute__((always_inline)) { b.s0[r][j] = x[(int)j]; });
        });
    }
}

// token i of a block: the decay, the write vector and k of the lane's rows
template <int RPL, typename E>
__device__ __forceinline__ void tok_rows(const ScanBwdParams &p, const Blk<RPL, E> &b, int i, float (&a)[RPL],
                                         float (&x)[RPL], float (&kk)[RPL]) {
    const float as = p.gate == 1 ? __expf(lane_val(b.gs, i)) : 1.f;
    const float bt = p.mode == 0 ? lane_val(b.bs, i) : 0.f;
    unroll<RPL>([&](auto r) __attribute__((always_inline)) {
        kk[r] = row_el<E, RPL>(b.k[i], r);
        a[r] = p.gate == 2 ? __expf(row_el<float, RPL>(b.g[i], r)) : as;
        x[r] = p.mode == 1 ? row_el<E, RPL>(b.w[i], r) : (p.mode == 0 ? kk[r] * bt : kk[r]);
    });
}

template <int DK>
__device__ __forceinline__ float *ckpt_at(float *base, const ScanBwdParams &p, int64_t slot, int h, int tile,
                                          int wv, int lane) {
    return base + ((slot * p.H + h) * p.n_tiles + tile) * (int64_t)(DK * p.TW) + (int64_t)(wv * 64 + lane) * (DK / 16);
}

// The two walks, one launch: workgroups [0, pairs * n_tiles) walk forward
// from h0, storing S at the entry of every block of CT tokens and u of every
// token; the others walk back from dht, storing dS (the gradient of the state
// at a block's exit) before each block, writing dv = dS^T x per token and dh0
// at the start.  The backward recurrence of dS reads only q, k, the
// write vector, the gate and do, so the two walks run side by side.
template <int DK, typename E>
__global__ void __launch_bounds__(256) scan_walks_kernel(ScanBwdParams p) {
    constexpr int RPL = DK / 64;
    constexpr int CT = SB_CT;
    using EL = Elem<E>;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t per_walk = (int64_t)p.geo.n_seqs * p.H * p.n_tiles;
    const bool back = blockIdx.x >= per_walk;
    const int64_t wg = back ? blockIdx.x - per_walk : blockIdx.x;
    const int tile = wg % p.n_tiles;
    const int pair = wg / p.n_tiles;
    const int s = pair / p.H, h = pair % p.H;
    const int H = p.H, DV = p.DV;
    int64_t bos, eos;
    seq_bounds(p.geo, s, bos, eos);
    const int64_t L = eos - bos;
    const int col0 = tile * p.TW + wv * 4;
    const int row0 = lane * RPL;
    const bool delta = p.mode != 2;
    const int64_t nblk = (L + CT - 1) / CT;
    const int64_t slot0 = bos / CT + s;
    // state tiles [n_seqs, H, DK, DV]: rows row0 + r, columns col0 .. col0 + 3
    const int64_t soff = ((int64_t)s * H + h) * DK * DV + (int64_t)row0 * DV + col0;
    float S[RPL][4];
    const float *init = back ? p.dht : p.h0;
    unroll<RPL>([&](auto r) __attribute__((always_inline)) {
        const f32x4 x = init ? ld4(init + soff + (int64_t)r * DV) : f32x4{0.f, 0.f, 0.f, 0.f};
        unroll<4>([&](auto j) __attribute__((always_inline)) { S[r][j] = x[(int)j]; });
    });

    if (!back) {
        auto fwd_block = [&](const Blk<RPL, E> &bk, int64_t b) __attribute__((always_inline)) {
            const int64_t t0 = b * CT;
            const int n = (int)(L - t0 < CT ? L - t0 : CT);
            float *c = ckpt_at<DK>(p.hs, p, slot0 + b, h, tile, wv, lane);
            unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                st4(c + r * 4, f32x4{S[r][0], S[r][1], S[r][2], S[r][3]});
            });
            const float vl = EL::to_f(bk.vr);
            unroll<CT>([&](auto i) __attribute__((always_inline)) {
                if (i < n) {
                    float a[RPL], x[RPL], kk[RPL], u[4];
                    tok_rows<RPL, E>(p, bk, i, a, x, kk);
                    unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                        unroll<4>([&](auto j) __attribute__((always_inline)) { S[r][j] *= a[r]; });
                    });
                    unroll<4>([&](auto j) __attribute__((always_inline)) { u[j] = lane_val(vl, 4 * i + j); });
                    if (delta) {
                        float pj[4];
                        unroll<4>([&](auto j) __attribute__((always_inline)) {
                            pj[j] = 0.f;
                            unroll<RPL>([&](auto r) __attribute__((always_inline)) { pj[j] += S[r][j] * kk[r]; });
                        });
                        wave_sum4(pj);
                        unroll<4>([&](auto j) __attribute__((always_inline)) { u[j] -= pj[j]; });
                        if (lane == 0)
                            st4(p.u + ((bos + t0 + i) * H + h) * DV + col0, f32x4{u[0], u[1], u[2], u[3]});
                    }
                    unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                        unroll<4>([&](auto j) __attribute__((always_inline)) { S[r][j] += x[r] * u[j]; });
                    });
                }
            });
        };
        Blk<RPL, E> A, B;
        if (nblk > 0) load_blk<RPL, E>(p, A, bos, L, 0, h, row0, lane, col0, false, nullptr);
        for (int64_t b = 0; b < nblk; b += 2) {
            load_blk<RPL, E>(p, B, bos, L, (b + 1) * CT, h, row0, lane, col0, false, nullptr);
            fwd_block(A, b);
            if (b + 1 < nblk) {
                load_blk<RPL, E>(p, A, bos, L, (b + 2) * CT, h, row0, lane, col0, false, nullptr);
                fwd_block(B, b + 1);
            }
        }
        return;
    }

    // the backward walk: S holds dS
    E *__restrict__ dvp = reinterpret_cast<E *>(p.dv);
    auto back_block = [&](const Blk<RPL, E> &bk, int64_t b) __attribute__((always_inline)) {
        const int64_t t0 = b * CT;
        const int n = (int)(L - t0 < CT ? L - t0 : CT);
        float *c = ckpt_at<DK>(p.dhs, p, slot0 + b, h, tile, wv, lane);
        unroll<RPL>([&](auto r) __attribute__((always_inline)) {
            st4(c + r * 4, f32x4{S[r][0], S[r][1], S[r][2], S[r][3]});
        });
        const float dl = EL::to_f(bk.dr);
        unroll<CT>([&](auto ii) __attribute__((always_inline)) {
            constexpr int i = CT - 1 - decltype(ii)::value;
            if (i < n) {
                float a[RPL], x[RPL], kk[RPL], dout[4], du[4];
                tok_rows<RPL, E>(p, bk, i, a, x, kk);
                unroll<4>([&](auto j) __attribute__((always_inline)) { dout[j] = lane_val(dl, 32 + 4 * i + j); });
                unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                    const float sq = p.scale * row_el<E, RPL>(bk.q[i], r);
                    unroll<4>([&](auto j) __attribute__((always_inline)) { S[r][j] += sq * dout[j]; });
                });
                unroll<4>([&](auto j) __attribute__((always_inline)) {
                    du[j] = 0.f;
                    unroll<RPL>([&](auto r) __attribute__((always_inline)) { du[j] += S[r][j] * x[r]; });
                });
                wave_sum4(du);
                if (lane == 0) {
                    const int64_t o = ((bos + t0 + i) * H + h) * DV + col0;
                    unroll<4>([&](auto j) __attribute__((always_inline)) { dvp[o + j] = EL::from_f(du[j]); });
                }
                unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                    unroll<4>([&](auto j) __attribute__((always_inline)) {
                        if (delta) S[r][j] -= kk[r] * du[j];
                        S[r][j] *= a[r];
                    });
                });
            }
        });
    };
    {
        Blk<RPL, E> A, B;
        if (nblk > 0) load_blk<RPL, E>(p, A, bos, L, (nblk - 1) * CT, h, row0, lane, col0, true, nullptr, false);
        for (int64_t b = nblk - 1; b >= 0; b -= 2) {
            load_blk<RPL, E>(p, B, bos, L, (b > 0 ? b - 1 : 0) * CT, h, row0, lane, col0, true, nullptr, false);
            back_block(A, b);
            if (b >= 1) {
                load_blk<RPL, E>(p, A, bos, L, (b > 1 ? b - 2 : 0) * CT, h, row0, lane, col0, true, nullptr, false);
                back_block(B, b - 1);
            }
        }
    }
    if (p.dh0) {
        unroll<RPL>([&](auto r) __attribute__((always_inline)) {
            st4(p.dh0 + soff + (int64_t)r * DV, f32x4{S[r][0], S[r][1], S[r][2], S[r][3]});
        });
    }
}

// The gradients of one block of CT tokens, all blocks in parallel: one
// workgroup per (checkpoint slot, head, tile).  It recomputes the block's
// states from the entry checkpoint and u, then walks the block back from the
// stored exit gradient, storing each wave's column sums of every token in its
// own LDS slice (no atomics: four waves adding to one row waited on the LDS),
// and writes the four slices' sum out as the tile's partials.
template <int DK, typename E>
__global__ void __launch_bounds__(256) scan_grad_kernel(ScanBwdParams p) {
    constexpr int RPL = DK / 64;
    constexpr int CT = SB_CT;
    using EL = Elem<E>;
    constexpr int NWG = 4;                            // waves per workgroup (16-column tiles)
    __shared__ float red[NWG][CT][4][DK];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nthr = blockDim.x;
    const int tile = blockIdx.x % p.n_tiles;
    const int64_t rest = blockIdx.x / p.n_tiles;
    const int h = (int)(rest % p.H);
    const int64_t slot = rest / p.H;
    const int H = p.H;
    // the sequence whose blocks hold this slot: the last s with bos(s) / CT + s <= slot
    int lo = 0, hi = p.geo.n_seqs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        int64_t b0, e0;
        seq_bounds(p.geo, mid, b0, e0);
        if (b0 / CT + mid <= slot) lo = mid; else hi = mid - 1;
    }
    const int s = lo;
    int64_t bos, eos;
    seq_bounds(p.geo, s, bos, eos);
    const int64_t L = eos - bos;
    const int64_t b = slot - (bos / CT + s);
    if (b < 0 || b * CT >= L) return;                 // a slot no block uses
    const int64_t t0 = b * CT;
    const int n = (int)(L - t0 < CT ? L - t0 : CT);
    const int col0 = tile * p.TW + wv * 4;
    const int row0 = lane * RPL;
    const bool delta = p.mode != 2;

    Blk<RPL, E> bk;
    load_blk<RPL, E>(p, bk, bos, L, t0, h, row0, lane, col0, true, ckpt_at<DK>(p.hs, p, slot, h, tile, wv, lane));
    float dS[RPL][4];
    {
        const float *c = ckpt_at<DK>(p.dhs, p, slot, h, tile, wv, lane);
        unroll<RPL>([&](auto r) __attribute__((always_inline)) {
            const f32x4 x = ld4(c + r * 4);
            unroll<4>([&](auto j) __attribute__((always_inline)) { dS[r][j] = x[(int)j]; });
        });
    }

    const float ul = delta ? bk.uf : EL::to_f(bk.vr);
    const float dl = EL::to_f(bk.dr);
    float st[CT][RPL][4];
    unroll<CT>([&](auto i) __attribute__((always_inline)) {
        if (i < n) {
            float a[RPL], x[RPL], kk[RPL];
            tok_rows<RPL, E>(p, bk, i, a, x, kk);
            unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                unroll<4>([&](auto j) __attribute__((always_inline)) {
                    const float prev = i == 0 ? bk.s0[r][j] : st[i == 0 ? 0 : i - 1][r][j];
                    st[i][r][j] = prev * a[r] + x[r] * lane_val(ul, 4 * i + j);
                });
            });
        }
    });
    unroll<CT>([&](auto ii) __attribute__((always_inline)) {
        constexpr int i = CT - 1 - decltype(ii)::value;
        if (i < n) {
            float a[RPL], x[RPL], kk[RPL], u[4], dout[4];
            tok_rows<RPL, E>(p, bk, i, a, x, kk);
            unroll<4>([&](auto j) __attribute__((always_inline)) {
                u[j] = lane_val(ul, 4 * i + j);
                dout[j] = lane_val(dl, 32 + 4 * i + j);
            });
            float pdq[RPL], pdk[RPL], pdx[RPL], pdg[RPL];
            unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                const float sq = p.scale * row_el<E, RPL>(bk.q[i], r);
                float aq = 0.f, ax = 0.f;
                unroll<4>([&](auto j) __attribute__((always_inline)) {
                    dS[r][j] += sq * dout[j];
                    aq += st[i][r][j] * dout[j];
                    ax += dS[r][j] * u[j];
                });
                pdq[r] = p.scale * aq;
                pdx[r] = ax;
            });
            float du[4];
            unroll<4>([&](auto j) __attribute__((always_inline)) {
                du[j] = 0.f;
                unroll<RPL>([&](auto r) __attribute__((always_inline)) { du[j] += dS[r][j] * x[r]; });
            });
            wave_sum4(du);
            unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                float ak = 0.f, ag = 0.f;
                unroll<4>([&](auto j) __attribute__((always_inline)) {
                    const float prev = i == 0 ? bk.s0[r][j] : st[i == 0 ? 0 : i - 1][r][j];
                    const float sb = prev * a[r];
                    if (delta) {
                        dS[r][j] -= kk[r] * du[j];
                        ak -= sb * du[j];
                    }
                    ag += dS[r][j] * sb;
                    dS[r][j] *= a[r];
                });
                pdk[r] = ak;
                pdg[r] = ag;
            });
            unroll<RPL>([&](auto r) __attribute__((always_inline)) {
                red[wv][i][0][row0 + r] = pdq[r];
                red[wv][i][1][row0 + r] = pdk[r];
                red[wv][i][2][row0 + r] = pdx[r];
                red[wv][i][3][row0 + r] = pdg[r];
            });
        }
    });
    __syncthreads();
    const int64_t plane = (int64_t)p.geo.n_tokens * H * DK;      // one (quantity, tile) partial
    for (int idx = tid; idx < n * 4 * DK; idx += nthr) {
        const int i = idx / (4 * DK), qn = (idx / DK) & 3, row = idx % DK;
        float sum = 0.f;
        unroll<NWG>([&](auto w) __attribute__((always_inline)) { sum += red[w][i][qn][row]; });
        p.part[(int64_t)(qn * p.n_tiles + tile) * plane + ((bos + t0 + i) * H + h) * DK + row] = sum;
    }
}

// one wave per (token, head): the tiles' partials summed, then
//   dq = P_q;  w given: dk = P_k, dw = P_x;  x = beta k: dk = P_k + beta P_x,
//   dbeta = k . P_x;  no delta: dk = P_x;  dg = P_g (per row) or its row sum
template <int DK, typename E>
__global__ void __launch_bounds__(256) scan_bwd_finish_kernel(ScanBwdParams p) {
    constexpr int RPL = DK / 64;
    using EL = Elem<E>;
    const int lane = threadIdx.x & 63;
    const int64_t rowi = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);     // token * H + head
    const int64_t nrows = p.geo.n_tokens * p.H;
    if (rowi >= nrows) return;
    const int64_t plane = nrows * DK;
    const int64_t off = rowi * DK + lane * RPL;
    float P[4][RPL];
    unroll<4>([&](auto qn) __attribute__((always_inline)) {
        unroll<RPL>([&](auto r) __attribute__((always_inline)) { P[qn][r] = 0.f; });
        for (int t = 0; t < p.n_tiles; ++t) {
            const float *src = p.part + (int64_t)(qn * p.n_tiles + t) * plane + off;
            unroll<RPL>([&](auto r) __attribute__((always_inline)) { P[qn][r] += src[r]; });
        }
    });
    E *dq = reinterpret_cast<E *>(p.dq) + off;
    E *dk = reinterpret_cast<E *>(p.dk) + off;
    float kk[RPL];
    load_f(reinterpret_cast<const E *>(p.k) + off, kk);
    const float b = p.mode == 0 ? p.beta[rowi] : 0.f;
    float db = 0.f, gs = 0.f;
    unroll<RPL>([&](auto r) __attribute__((always_inline)) {
        dq[r] = EL::from_f(P[0][r]);
        if (p.mode == 1) {
            dk[r] = EL::from_f(P[1][r]);
            reinterpret_cast<E *>(p.dw)[off + r] = EL::from_f(P[2][r]);
        } else if (p.mode == 0) {
            dk[r] = EL::from_f(P[1][r] + b * P[2][r]);
            db += kk[r] * P[2][r];
        } else {
            dk[r] = EL::from_f(P[2][r]);
        }
        if (p.gate == 2) p.dg[off + r] = P[3][r];
        gs += P[3][r];
    });
    if (p.mode == 0) {
        db = wave_sum(db);
        if (lane == 0) p.dbeta[rowi] = db;
    }
    if (p.gate == 1) {
        gs = wave_sum(gs);
        if (lane == 0) p.dg[rowi] = gs;
    }
}

template <int DK, typename E>
hipError_t launch(const ScanBwdParams &p, hipStream_t stream) {
    const int64_t pairs = (int64_t)p.geo.n_seqs * p.H;
    if (p.TW != 16) return hipErrorInvalidValue;               // the grad kernel's LDS holds 4 waves
    if (pairs > 0) {
        const dim3 blk(64 * (p.TW / 4));
        scan_walks_kernel<DK, E><<<dim3((unsigned)(2 * pairs * p.n_tiles)), blk, 0, stream>>>(p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t slots = scan_bwd_ckpt_slots(p.geo.n_tokens, p.geo.n_seqs);
        scan_grad_kernel<DK, E><<<dim3((unsigned)(slots * p.H * p.n_tiles)), blk, 0, stream>>>(p);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const int64_t nrows = p.geo.n_tokens * p.H;
    if (nrows > 0) {
        scan_bwd_finish_kernel<DK, E><<<dim3((unsigned)((nrows + 3) / 4)), dim3(256), 0, stream>>>(p);
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace

hipError_t scan_bwd(int dtype, int dk, const ScanBwdParams &p, hipStream_t stream) {
    if (dk == 128) {
        if (dtype == 0) return launch<128, float>(p, stream);
        if (dtype == 1) return launch<128, __bf16>(p, stream);
        return launch<128, _Float16>(p, stream);
    }
    if (dtype == 0) return launch<64, float>(p, stream);
    if (dtype == 1) return launch<64, __bf16>(p, stream);
    return launch<64, _Float16>(p, stream);
}

}  // namespace vgdr

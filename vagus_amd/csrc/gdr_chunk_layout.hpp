// Layout of the per-(chunk, head) blocks chunk_prep_kernel leaves in the
// workspace, the sequence geometry helpers and the LDS transpose read, shared
// by the forward chunk kernels (gdr_chunk.hip) and the backward ones
// (gdr_chunk_bwd.hip).
#pragma once

#include "gdr_common.hpp"
#include "gdr_kernels.hpp"

namespace vgdr {

// Fragment order of a CH x CH block of 16 x 16 tiles, by tile pairs: the
// eight elements lane 16 g + m contributes to one 16x16x32 MFMA over k-blocks
// (2 q, 2 q + 1), i.e. elements (16 I + m, 16 (2 q) + 4 g + j) and
// (16 I + m, 16 (2 q + 1) + 4 g + j), j = 0..3, are contiguous, and a
// wavefront reads a tile pair as one contiguous run of 64 * 8 elements.
// frag_pair_pos gives the start of a lane's eight; frag_pos the four of one tile.
template <int NB>
__device__ __forceinline__ int frag_pair_pos(int I, int q, int lane) {
    static_assert(NB % 2 == 0, "tiles are paired");
    return ((I * (NB / 2) + q) * 64 + lane) * 8;
}
template <int NB>
__device__ __forceinline__ int frag_pos(int I, int kb, int lane) {
    return frag_pair_pos<NB>(I, kb >> 1, lane) + (kb & 1) * 4;
}

// The per-(chunk slot, head) block chunk_prep leaves in the workspace: TE and
// A (CH x CH each, element type, tile-pair fragment order), then
//   scalar gate (or none), with G_t = exp(gamma_t), Gend_t = exp(gamma_C - gamma_t)
//       and the rows' L2-norm factors rk_t, rq_t (1 unless the norm is fused):
//       GX_t = G_t rk_t (for X), GO_t = scale G_t rq_t (for O), GE_t = Gend_t rk_t
//       (for the state update; 0 past a partial chunk's end), CH floats each,
//       then Gc = exp(gamma_C) and three floats of padding;
//   per-channel gate, 16-bit elements (VEC): the gated tiles K*G, scale Q*G and
//       K*Gend (CH x DK each, element type, unpadded rows; K*G and K*Gend in the
//       paired-column order of KQRows, scale Q*G in natural column order), then
//       Gc = exp(gamma_C) (DK floats).
// Blocks are 16-byte multiples.
template <typename E, int CH, int DK, int GATE>
struct ChunkBlock {
    static constexpr bool VEC = GATE == 2 && sizeof(E) == 2;
    static constexpr int TEA = 2 * CH * CH;                                   // elements of TE and A
    static constexpr int TILES = VEC ? 3 * CH * DK : 0;                       // elements of the gated tiles
    static constexpr int GOFF = (TEA + TILES) * (int)sizeof(E);               // byte offset of the floats
    static constexpr int FLOATS = VEC ? DK : 3 * CH + 4;
    static constexpr int BYTES = GOFF + FLOATS * 4;
    static_assert(BYTES % 16 == 0 && GOFF % 16 == 0, "blocks are copied in 16-byte units");
};

__device__ __forceinline__ void seq_bounds(const SeqGeom &g, int seq, int64_t &bos, int64_t &eos) {
    if (g.cu) {
        int64_t a = g.cu[seq], b = g.cu[seq + 1];
        a = a < 0 ? 0 : (a > g.n_tokens ? g.n_tokens : a);
        b = b < a ? a : (b > g.n_tokens ? g.n_tokens : b);
        bos = a;
        eos = b;
    } else {
        bos = (int64_t)seq * g.T;
        eos = bos + g.T;
    }
}

__device__ __forceinline__ int64_t chunk_base(const SeqGeom &g, int seq) {
    return g.cu ? (int64_t)g.chunk_offs[seq] : (int64_t)seq * g.chunks_per_seq;
}

template <typename E>
__device__ __forceinline__ typename Elem<E>::frag gfrag(const E *p) {
    return *reinterpret_cast<const typename Elem<E>::frag *>(p);
}

// The chunked backward's per-(chunk, head) state checkpoints (dk x dv in the
// element type) are stored in C-layout fragment order: for column block cb
// (columns 16 cb .. 16 cb + 15) and key block kt, lane l = 16 g + r holds rows
// 16 kt + 4 g .. + 3 of column 16 cb + r, the four entries at ckpt_pos(cb, kt,
// l).  A wavefront that owns a column block writes one contiguous 512-element
// run per key block, and the column blocks of a dv range are contiguous.
template <int DK>
__device__ __forceinline__ int64_t ckpt_pos(int cb, int kt, int lane) {
    return ((int64_t)(cb * (DK / 16) + kt) * 64 + lane) * 4;
}

// gfx950 ds_read_b64_tr_b16: within each 16-lane group, source lane s gives the
// address of 4 consecutive 16-bit elements, and result lane d receives element
// d % 4 of source lanes d / 4 + 4 i (i = 0..3).  With source lane s pointing at
// row k0 + s / 4, columns c0 + 4 (s % 4) of a row-major tile, lane d receives
// rows k0 .. k0 + 3 of column c0 + d: the C-layout / B-operand fragment of the
// tile, or the A-operand fragment of its transpose, read straight from
// row-major storage.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s16x4 lds_tr16(const void *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)const_cast<void *>(p));
}
template <typename E>
__device__ __forceinline__ typename Elem<E>::frag ld_tr(const E *p) {
    return __builtin_bit_cast(typename Elem<E>::frag, lds_tr16(p));
}

}  // namespace vgdr

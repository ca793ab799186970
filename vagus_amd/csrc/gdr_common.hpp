// Shared device helpers for the gfx950 gated delta-rule kernels.
//
// MFMA fragment convention used by every product in this library
// ------------------------------------------------------------------
// A 16x16 output tile C = A (16 x K) * B (K x 16) is accumulated by one
// wavefront.  Lane l = 16*g + r (g = l / 16 in 0..3, r = l % 16) holds
//     C[4g + j][r]                        j = 0..3        ("C layout")
// The contraction index K is cut into k-blocks of 16.  For k-block kb a lane
// contributes the four indices 16*kb + 4g + j (j = 0..3):
//     A operand: A[r][16kb + 4g + j]      (row r of A, four consecutive k)
//     B operand: B[16kb + 4g + j][r]      (column r of B, four consecutive k)
// bf16 / fp16 use v_mfma_f32_16x16x32_{bf16,f16}, which consumes two k-blocks
// per instruction (its 8 k-slots of lane group g are taken as
// {16kb0 + 4g + 0..3, 16kb1 + 4g + 0..3}); fp32 uses four v_mfma_f32_16x16x4f32,
// instruction j taking k-slot g = index 16kb + 4g + j.  A and B use the same
// slot-to-index map, so the permutation cancels in the sum.
//
// The point of the convention: a C-layout tile *is* a B operand (its rows
// become the contraction index), so a product's accumulator feeds the next
// product straight from registers.  The recurrent state S lives in C-layout
// accumulators for the whole sequence.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace vgdr {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// element traits
// ---------------------------------------------------------------------------
template <typename E> struct Elem;

template <> struct Elem<float> {
    using frag = f32x4;                       // one k-block share of a lane
    static constexpr int pad = 4;             // LDS row padding (elements)
    static constexpr float gate_range = 60.f; // KDA sub-block factorisation limit (nats)
    __device__ static __forceinline__ float to_f(float x) { return x; }
    __device__ static __forceinline__ float from_f(float x) { return x; }
    __device__ static __forceinline__ frag cvt(f32x4 x) { return x; }
    __device__ static __forceinline__ f32x4 tof(frag x) { return x; }
};

template <> struct Elem<__bf16> {
    using frag = bf16x4;
    using frag2 = bf16x8;                     // both k-blocks of one 16x16x32 MFMA
    static constexpr int pad = 4;
    static constexpr float gate_range = 60.f;
    __device__ static __forceinline__ float to_f(__bf16 x) { return (float)x; }
    __device__ static __forceinline__ __bf16 from_f(float x) { return (__bf16)x; }
    __device__ static __forceinline__ frag cvt(f32x4 x) {
        return frag{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]};
    }
    __device__ static __forceinline__ f32x4 tof(frag x) {
        return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
    }
    __device__ static __forceinline__ frag2 cvt2(f32x4 a, f32x4 b) {
        return frag2{(__bf16)a[0], (__bf16)a[1], (__bf16)a[2], (__bf16)a[3],
                     (__bf16)b[0], (__bf16)b[1], (__bf16)b[2], (__bf16)b[3]};
    }
};

template <> struct Elem<_Float16> {
    using frag = f16x4;
    using frag2 = f16x8;
    static constexpr int pad = 4;
    static constexpr float gate_range = 8.f;  // fp16 overflows past e^11
    __device__ static __forceinline__ float to_f(_Float16 x) { return (float)x; }
    __device__ static __forceinline__ _Float16 from_f(float x) { return (_Float16)x; }
    __device__ static __forceinline__ frag cvt(f32x4 x) {
        return frag{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
    }
    __device__ static __forceinline__ f32x4 tof(frag x) {
        return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
    }
    __device__ static __forceinline__ frag2 cvt2(f32x4 a, f32x4 b) {
        return frag2{(_Float16)a[0], (_Float16)a[1], (_Float16)a[2], (_Float16)a[3],
                     (_Float16)b[0], (_Float16)b[1], (_Float16)b[2], (_Float16)b[3]};
    }
};

// ---------------------------------------------------------------------------
// MFMA over k-blocks
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma_kb1(f32x4 a, f32x4 b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
    return c;
}
__device__ __forceinline__ f32x4 mfma_kb2(f32x4 a0, f32x4 b0, f32x4 a1, f32x4 b1, f32x4 c) {
    return mfma_kb1(a1, b1, mfma_kb1(a0, b0, c));
}

__device__ __forceinline__ f32x4 mfma_kb2(bf16x4 a0, bf16x4 b0, bf16x4 a1, bf16x4 b1, f32x4 c) {
    bf16x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
    bf16x8 b = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_kb1(bf16x4 a, bf16x4 b, f32x4 c) {
    const bf16x4 z = {};
    return mfma_kb2(a, b, z, z, c);
}

__device__ __forceinline__ f32x4 mfma_kb2(f16x4 a0, f16x4 b0, f16x4 a1, f16x4 b1, f32x4 c) {
    f16x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
    f16x8 b = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_kb1(f16x4 a, f16x4 b, f32x4 c) {
    const f16x4 z = {};
    return mfma_kb2(a, b, z, z, c);
}

// one 16x16x32 MFMA on operands that already hold both k-blocks (frag2)
__device__ __forceinline__ f32x4 mfma_pair(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_pair(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// c += sum over k-blocks kb in [0, n) of A(kb) * B(kb); fa / fb return the
// lane's fragment of k-block kb.
template <typename FA, typename FB>
__device__ __forceinline__ f32x4 contract(f32x4 c, int n, FA fa, FB fb) {
    int kb = 0;
#pragma unroll
    for (; kb + 1 < n; kb += 2) c = mfma_kb2(fa(kb), fb(kb), fa(kb + 1), fb(kb + 1), c);
    if (kb < n) c = mfma_kb1(fa(kb), fb(kb), c);
    return c;
}

// LDS fragment access: four consecutive elements, aligned to their size.
template <typename E>
__device__ __forceinline__ typename Elem<E>::frag ld_frag(const E *p) {
    return *reinterpret_cast<const typename Elem<E>::frag *>(p);
}
template <typename E>
__device__ __forceinline__ void st_frag(E *p, typename Elem<E>::frag x) {
    *reinterpret_cast<typename Elem<E>::frag *>(p) = x;
}

__device__ __forceinline__ f32x4 ld4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
__device__ __forceinline__ void st4(float *p, f32x4 x) { *reinterpret_cast<f32x4 *>(p) = x; }

__device__ __forceinline__ f32x4 exp4(f32x4 x) {
    return f32x4{__expf(x[0]), __expf(x[1]), __expf(x[2]), __expf(x[3])};
}

template <typename T> __host__ __device__ constexpr T cmax(T a, T b) { return a > b ? a : b; }

// Workgroup barrier that orders LDS traffic only: waits for this wave's LDS
// operations, then s_barrier.  Unlike __syncthreads() it does not wait for
// outstanding global memory operations, so loads still in flight (an
// asynchronous copy into the other double-buffer slot, a state tile) keep
// flowing across it.  The memory clobber stops the compiler from moving memory
// accesses across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Buffer access to one contiguous block [base, base + bytes): a load or store
// takes a 32-bit per-lane offset and a scalar offset instead of a 64-bit address
// per lane (two VGPRs per access in flight), and an access outside the block
// reads zeros or is dropped.  The resource's last word is the gfx9 format word;
// CPOL_NT is the non-temporal bit of the cache policy (gfx94x, gfx950).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int CPOL_NT = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f32x4 buffer_load_nt4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, CPOL_NT));
}
__device__ __forceinline__ void buffer_store_nt4(f32x4 x, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), r, (int)voff, (int)soff, CPOL_NT);
}
// Stores that need no branch: a lane (or a wave, with a zero-byte resource)
// whose store must not happen gets an offset outside the block.  A store under
// a branch makes the join wait for every memory operation in flight (the wave
// cannot know which path issued how many), stores included.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
template <typename F8>
__device__ __forceinline__ void buffer_store_8b(F8 x, __amdgpu_buffer_rsrc_t r, uint32_t voff) {
    static_assert(sizeof(F8) == 8, "an 8-byte fragment");
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, x), r, (int)voff, 0, 0);
}
template <typename E2>
__device__ __forceinline__ void buffer_store_2b(E2 x, __amdgpu_buffer_rsrc_t r, uint32_t voff) {
    static_assert(sizeof(E2) == 2, "a 16-bit element");
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, x), r, (int)voff, 0, 0);
}

// the reference's producer activations (linear_attention.py:703-706, :719-736)
// 1 / (1 + e^-x) with the hardware reciprocal (v_rcp_f32, about 1 ulp): an IEEE
// division costs a dozen instructions, which made the SiLU of the streaming
// conv and epilogue kernels bound by the vector ALU rather than by HBM
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// torch.nn.functional.softplus (beta 1, threshold 20)
__device__ __forceinline__ float softplusf_(float x) { return x > 20.f ? x : log1pf(__expf(x)); }
// gate activation of the per-channel gate from its pre-activation f
__device__ __forceinline__ float gate_activation(float f, float a_log, float dt, int lb_set, float lb) {
    const float a = __expf(a_log), z = f + dt;
    return lb_set ? lb * sigmoidf_(a * z) : -a * softplusf_(z);
}

// 16-byte global access
struct alignas(16) Vec16 { uint32_t w[4]; };
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N - 1>{}).
// Register arrays indexed inside f are indexed by constants from the start:
// a `#pragma unroll` loop is unrolled only after the alloca promotion pass,
// which places a dynamically indexed array in LDS or scratch instead.
template <typename F, int... I>
__device__ __forceinline__ void unroll_seq(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unroll(F &&f) {
    unroll_seq(f, std::make_integer_sequence<int, N>{});
}

// ---- cross-lane sums and scans in VALU (DPP) ---------------------------------
// A __shfl_* is a round trip through the LDS crossbar (ds_bpermute_b32); these
// read the neighbour lane through a DPP operand of the add instead.
// dpp_f<CTRL>(x): x from the lane the DPP control names (row_ror, row_shr,
// row_bcast ..); a lane whose source lies outside its row, or whose row
// ROW_MASK leaves out, reads 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xf,
                                                                 false));
}
// the sum over the 16 lanes of x's row (lanes 16 m .. 16 m + 15), in every lane
// of the row (each lane adds in its own order: lanes may differ in the last bit)
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp_f<0x128>(x);                                     // row_ror:8
    x += dpp_f<0x124>(x);                                     // row_ror:4
    x += dpp_f<0x122>(x);                                     // row_ror:2
    x += dpp_f<0x121>(x);                                     // row_ror:1
    return x;
}
// the sum over the wave, in every lane: the rows' sums, the two row broadcasts
// carry rows 0 .. 2 into row 3, and lane 63's value is read out
__device__ __forceinline__ float wave_sum64(float x) {
    x = row_sum16(x);
    x += dpp_f<0x142, 0xa>(x);                                // row_bcast:15 into rows 1 and 3
    x += dpp_f<0x143, 0xc>(x);                                // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}
// inclusive prefix sum over lanes 0 .. l: row shifts 1, 2, 4, 8, then the rows'
// totals carried forward by the two row broadcasts
__device__ __forceinline__ float wave_scan(float x) {
    x += dpp_f<0x111>(x);                                     // row_shr:1
    x += dpp_f<0x112>(x);                                     // row_shr:2
    x += dpp_f<0x114>(x);                                     // row_shr:4
    x += dpp_f<0x118>(x);                                     // row_shr:8
    x += dpp_f<0x142, 0xa>(x);                                // row_bcast:15
    x += dpp_f<0x143, 0xc>(x);                                // row_bcast:31
    return x;
}
// suffix sum over lanes l .. 63: the total less the exclusive prefix
__device__ __forceinline__ float wave_suffix(float x) {
    const float inc = wave_scan(x);
    const float tot = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inc), 63));
    return tot - (inc - x);
}

}  // namespace vgdr

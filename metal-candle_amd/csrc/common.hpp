// Shared device helpers for the gfx950 kernels: bf16 conversion, wave64
// reductions over DPP, 16-byte vector types, MFMA operand types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mc {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even fp32 -> bf16 (gfx950 lowers this to v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    __bf16 b = static_cast<__bf16>(f);
    return __builtin_bit_cast(uint16_t, b);
}
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
// Two floats to a bf16 pair (lo in bits 0-15), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2v v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}
// Eight floats to an MFMA bf16 operand, element e from v[e].
__device__ __forceinline__ bf16x8 pack_bf16x8(const float* v) {
    const u32x4 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                     pack_bf16x2(v[6], v[7])};
    return __builtin_bit_cast(bf16x8, w);
}

// 2^x with the hardware instruction (v_exp_f32), without the library's
// rescaling for results below 2^-126, which come out as 0 here. Used where
// the argument is a max-shifted score, so such terms are negligible in any
// sum they enter; exp2(-inf) = 0.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Storage-type traits: float or bf16 (stored as uint16_t bit patterns).
template <typename T> struct Elem;
template <> struct Elem<float> {
    static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<uint16_t> {
    static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
    static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};

// 16-byte vectors: 4 floats or 8 bf16.
template <typename T> struct Vec16;
template <> struct Vec16<float> {
    static constexpr int N = 4;
    static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
        float4 q = *reinterpret_cast<const float4*>(p);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
    static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
};
template <> struct Vec16<uint16_t> {
    static constexpr int N = 8;
    static __device__ __forceinline__ void load(const uint16_t* p, float (&v)[8]) {
        uint4 q = *reinterpret_cast<const uint4*>(p);
        v[0] = bf16_lo(q.x); v[1] = bf16_hi(q.x); v[2] = bf16_lo(q.y); v[3] = bf16_hi(q.y);
        v[4] = bf16_lo(q.z); v[5] = bf16_hi(q.z); v[6] = bf16_lo(q.w); v[7] = bf16_hi(q.w);
    }
    static __device__ __forceinline__ void store(uint16_t* p, const float (&v)[8]) {
        uint4 q;
        q.x = pack_bf16x2(v[0], v[1]); q.y = pack_bf16x2(v[2], v[3]);
        q.z = pack_bf16x2(v[4], v[5]); q.w = pack_bf16x2(v[6], v[7]);
        *reinterpret_cast<uint4*>(p) = q;
    }
};

// ------------------------------------------------------ wave reductions
// Butterfly over the 64 lanes: DPP quad_perm [1,0,3,2] and [2,3,0,1], then
// row_half_mirror and row_mirror (lane i <-> 7-i / 15-i, which pairs every
// quad / half-row with its partner once the lanes within it agree), then two
// ds_bpermute exchanges across the 16-lane rows. Every lane ends with the
// full result; the combination order is fixed, so results are reproducible.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    v = fmaxf(v, __shfl_xor(v, 16, kWave));
    v = fmaxf(v, __shfl_xor(v, 32, kWave));
    return v;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// ---------------------------------------------------- buffer resources
// Raw buffer resource (gfx9 layout, stride 0) over [base, base + bytes):
// loads at byte offsets >= num_records return zeros (loads into LDS write
// zeros) and stores there are dropped, which gives branch-free bounds
// handling. kOOB is an offset that is always out of range. num_records is
// 32-bit: callers keep every offset below 2^31 by basing the resource at
// the block of rows a workgroup touches.
constexpr uint32_t kOOB = 0x80000000u;
// Cache-policy bits of a buffer store (the builtins' aux operand, gfx950
// encoding): nt, a non-temporal (streaming) store that leaves no dirty line
// in L2. Used for outputs written as whole 128-byte lines and not read again
// by the kernel that writes them.
constexpr int kStoreNT = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    const int n = bytes <= 0 ? 0 : bytes >= 0x7fffffff ? 0x7fffffff : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
__device__ __forceinline__ i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

// 16-byte vectors of T (4 floats or 8 bf16) at a byte offset of a buffer
// resource, converted to / from fp32. Out-of-range offsets load zeros and
// drop the store, so callers select offsets instead of branching.
template <typename T> struct BVec;
template <> struct BVec<float> {
    static constexpr int N = 4;
    static __device__ __forceinline__ void unpack(const i32x4& q, float (&v)[4]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __int_as_float(q[e]);
    }
    static __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&v)[4]) {
        unpack(buf_load16(r, off), v);
    }
    static __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&v)[4]) {
        const i32x4 q = {__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]), __float_as_int(v[3])};
        __builtin_amdgcn_raw_buffer_store_b128(q, r, (int)off, 0, 0);
    }
    // the same as a non-temporal store (kStoreNT)
    static __device__ __forceinline__ void store_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&v)[N]) {
        i32x4 q;
        if constexpr (N == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = __float_as_int(v[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = (int)pack_bf16x2(v[2 * e], v[2 * e + 1]);
        }
        __builtin_amdgcn_raw_buffer_store_b128(q, r, (int)off, 0, kStoreNT);
    }
};
template <> struct BVec<uint16_t> {
    static constexpr int N = 8;
    static __device__ __forceinline__ void unpack(const i32x4& q, float (&v)[8]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = bf16_lo((uint32_t)q[e]);
            v[2 * e + 1] = bf16_hi((uint32_t)q[e]);
        }
    }
    static __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&v)[8]) {
        unpack(buf_load16(r, off), v);
    }
    static __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&v)[8]) {
        const i32x4 q = {(int)pack_bf16x2(v[0], v[1]), (int)pack_bf16x2(v[2], v[3]), (int)pack_bf16x2(v[4], v[5]),
                         (int)pack_bf16x2(v[6], v[7])};
        __builtin_amdgcn_raw_buffer_store_b128(q, r, (int)off, 0, 0);
    }
    // the same as a non-temporal store (kStoreNT)
    static __device__ __forceinline__ void store_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&v)[N]) {
        i32x4 q;
        if constexpr (N == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = __float_as_int(v[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = (int)pack_bf16x2(v[2 * e], v[2 * e + 1]);
        }
        __builtin_amdgcn_raw_buffer_store_b128(q, r, (int)off, 0, kStoreNT);
    }
};

// ----------------------------------------------------------- LDS DMA
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// LDS tile layout: rows of BK bf16 (2 BK bytes, no padding), CPR = BK/8
// 16-byte chunks per row; chunk c of row r sits in slot
// c ^ ((r / (128/BK)) % CPR). A 256-byte bank window holds 128/BK rows, so a
// 16-lane group touches 16 distinct 16-byte bank groups both when the loads
// write whole rows and when the MFMA fragment reads walk down 16 rows of one
// chunk column.
template <int BK>
__device__ __forceinline__ int swz(int r, int c) {
    return c ^ ((r / (128 / BK)) % (BK / 8));
}

// One buffer_load_dwordx4 ... lds: 64 lanes x 16 B to LDS bytes
// [lds_byte, lds_byte + 1 KB), lane l -> lds_byte + 16 l (M0 holds the LDS
// base). Issued from inline asm so that the compiler's wait-count pass does
// not see an LDS write it cannot place, which makes it wait for every such
// load before any LDS read; the kernel waits for these loads itself
// (wait_vmcnt + barrier) before the stage they fill is read.
// M0 is a register the compiler reserves, so clang notes that its clobber
// may not be honoured. The kernels that use this helper contain no
// compiler-generated M0 use (gfx9 DS instructions do not read it): every M0
// write in their ISA is one of these asm blocks, each immediately followed by
// the load that reads it.
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_byte, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_byte), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

// dma16 with a wave-uniform byte offset in soffset (added to the address
// outside the VGPR offset): loops that advance along a row pass the advance
// here and keep each lane's VGPR offset fixed.
__device__ __forceinline__ void dma16_s(i32x4 rsrc, uint32_t lds_byte, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_byte), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}

// Loads rows [0, ROWS) x BK columns (k = kb .. kb+BK-1) of one operand tile
// into the swizzled layout at lds_byte: a load moves RPI = 512/BK rows; each
// wave issues ROWS/RPI/waves of them, split over PARTS calls (part p issues
// loads p, p + PARTS, ...); lane l fetches the global chunk that the swizzle
// places at row RPI i + l / CPR, slot l % CPR. Chunks at k >= ks load as
// zeros.
template <int ROWS, int NT, int BK, int PARTS = 1>
__device__ __forceinline__ void dma_tile(i32x4 r, uint32_t lds_byte, uint32_t ld, uint32_t kb, uint32_t ks,
                                         int tid, int part = 0) {
    constexpr int CPR = BK / 8, RPI = 64 / CPR;
    static_assert(ROWS % (RPI * (NT / 64)) == 0, "rows per wave");
    constexpr int PER_WAVE = ROWS / RPI / (NT / 64);
    static_assert(PER_WAVE >= 1, "rows per wave");
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
        if (j % PARTS != part) continue;  // part p issues loads p, p + PARTS, ...
        const int blk = wave * PER_WAVE + j;
        const int row = blk * RPI + lane / CPR;
        const uint32_t k = kb + 8u * (uint32_t)swz<BK>(row, lane % CPR);
        const uint32_t off = k < ks ? ((uint32_t)row * ld + k) * 2u : kOOB;
        // the LDS address is wave-uniform: make it scalar for M0
        dma16(r, __builtin_amdgcn_readfirstlane(lds_byte + (uint32_t)blk * 1024u), off);
    }
}

__device__ __forceinline__ i32x4 rsrc_words(const void* base, int64_t bytes) {
    const int n = bytes <= 0 ? 0 : bytes >= 0x7fffffff ? 0x7fffffff : (int)bytes;
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4 r;
    r[0] = (int)(uint32_t)a;
    r[1] = (int)(uint32_t)(a >> 32) & 0xffff;  // stride 0
    r[2] = n;
    r[3] = 0x00020000;
    return r;
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wave index within the workgroup as a scalar (wave-uniform) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// ------------------------------------------------- workgroup reductions
// Over every wave of a workgroup of up to kMaxWaves waves: each wave's
// butterfly result goes to red[wave]; after the barrier every thread combines
// the slots in wave order, so all threads get the same, reproducible value.
// A slot array must not be written again until every thread has read it:
// callers give each reduction of a phase its own array, with a barrier
// between reuses.
constexpr int kMaxWaves = 16;
__device__ __forceinline__ float wg_sum(float v, float* red) {
    v = wave_sum(v);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    const int nw = (int)(blockDim.x >> 6);
    float t = red[0];
    for (int k = 1; k < nw; ++k) t += red[k];
    return t;
}
__device__ __forceinline__ float wg_max(float v, float* red) {
    v = wave_max(v);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    const int nw = (int)(blockDim.x >> 6);
    float t = red[0];
    for (int k = 1; k < nw; ++k) t = fmaxf(t, red[k]);
    return t;
}

// 16-byte load of base[off .. off+8) (bf16) or base[off .. off+4) (fp32) that
// yields zeros when !ok. The load itself is unconditional from an in-bounds
// address (base[0] when !ok) and the zero is a value select: a conditional
// load written as `ok ? *p : zero` is lowered to a load through a selected
// pointer to a stack copy of `zero`, i.e. flat loads and scratch traffic.
template <typename T>
__device__ __forceinline__ uint4 load16(const T* base, int64_t off, bool ok) {
    const uint4 v = *reinterpret_cast<const uint4*>(base + (ok ? off : 0));
    return ok ? v : make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace mc

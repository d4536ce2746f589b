// Shared device helpers and the C-ABI error plumbing of the sfnx_amd library (gfx950, wave64).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "../../include/sfnx_moe.h"

namespace sfnx {

constexpr int WAVE = 64;
constexpr int Q4K_BYTES = 144, Q5K_BYTES = 176, Q40_BYTES = 18, Q51_BYTES = 24, Q80_BYTES = 34, Q81_BYTES = 36;

// ------------------------------------------------------------------------------------------------ errors
void set_error(const std::string& msg);
// runs f, mapping a thrown error (or a failed launch) to a negative status and the thread's message
template <typename F> int guarded(const char* what, F&& f) {
    try {
        f();
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) throw std::runtime_error(std::string("launch failed: ") + hipGetErrorString(e));
        return 0;
    } catch (const std::exception& ex) {
        set_error(std::string(what) + ": " + ex.what());
        return -1;
    }
}
// the same for host-only work (no launch to check, and no GPU needed)
template <typename F> int guarded_host(const char* what, F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& ex) {
        set_error(std::string(what) + ": " + ex.what());
        return -1;
    }
}
inline void require(bool ok, const char* msg) {
    if (!ok) throw std::runtime_error(msg);
}
inline void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
inline hipStream_t stream_of(void* st) { return reinterpret_cast<hipStream_t>(st); }

// ------------------------------------------------------------------------------------------------ device helpers
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// the value of lane (this lane xor O), O a power of two below 64, without the LDS crossbar: DPP quad permutes for 1
// and 2, row shifts for 4, a row rotation for 8, and gfx950's permlane swaps across rows for 16 and 32
template <int CTRL, int ROWS = 0xf> __device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROWS, 0xf, false);
}
template <int O> __device__ __forceinline__ int lane_xor(int v) {
    if constexpr (O == 1) {
        return dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    } else if constexpr (O == 2) {
        return dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    } else if constexpr (O == 4) {
        const int up = dpp_mov<0x104>(v), down = dpp_mov<0x114>(v);   // row_shl:4 (lane + 4), row_shr:4 (lane - 4)
        return (__lane_id() & 4) ? down : up;
    } else if constexpr (O == 8) {
        return dpp_mov<0x128>(v);   // row_ror:8
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned) v, (unsigned) v, false, false);
        return (int) ((__lane_id() & 16) ? r[0] : r[1]);
    } else {
        static_assert(O == 32, "lane_xor: O in 1 .. 32");
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned) v, (unsigned) v, false, false);
        return (int) ((__lane_id() & 32) ? r[0] : r[1]);
    }
}
template <int O> __device__ __forceinline__ float lane_xor(float v) { return __int_as_float(lane_xor<O>(__float_as_int(v))); }

// lanes xor-reduced within groups of G (G a power of two <= 64): the tree every lane of a group ends with, partner
// values exactly those of __shfl_xor
template <int G, typename T, typename F> __device__ __forceinline__ T group_reduce(T v, F op) {
    if constexpr (G >= 64) v = op(v, lane_xor<32>(v));
    if constexpr (G >= 32) v = op(v, lane_xor<16>(v));
    if constexpr (G >= 16) v = op(v, lane_xor<8>(v));
    if constexpr (G >= 8) v = op(v, lane_xor<4>(v));
    if constexpr (G >= 4) v = op(v, lane_xor<2>(v));
    if constexpr (G >= 2) v = op(v, lane_xor<1>(v));
    return v;
}
template <int G> __device__ __forceinline__ float group_sum(float v) {
    return group_reduce<G>(v, [](float a, float b) { return a + b; });
}
template <int G> __device__ __forceinline__ float group_max(float v) {
    return group_reduce<G>(v, [](float a, float b) { return fmaxf(a, b); });
}
template <int G> __device__ __forceinline__ int group_isum(int v) {
    return group_reduce<G>(v, [](int a, int b) { return a + b; });
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// 1 / sqrt(mean(x^2) + eps) of a row of H values (H % 256 == 0) by one wavefront, in the router's partition: lane l
// sums the squares of its float4 chunks l, l + 64, ... in order (fmaf), then a xor butterfly; every lane returns the
// same value.  rms_from_sum finishes it from the lane sums.
__device__ __forceinline__ float rms_lane_add(float4 v, float ss) {
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    return fmaf(v.w, v.w, ss);
}
__device__ __forceinline__ float rms_from_sum(float ss, int H, float eps) {
    ss = group_sum<WAVE>(ss);
    return 1.0f / sqrtf(ss / (float) H + eps);
}
__device__ __forceinline__ float wave_rms_scale(const float* x, int H, int lane, float eps) {
    float ss = 0.f;
    for (int c = lane; c < H / 4; c += WAVE) ss = rms_lane_add(reinterpret_cast<const float4*>(x)[c], ss);
    return rms_from_sum(ss, H, eps);
}

// silu and sigmoid as the reference writes them (src/kernels.cu:46-47), exp by the device library
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigm_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// get_scale_min_k4 on the 16-byte header held in h (bytes 4..15 are the scales; src/moe_q4k.cuh:15-23)
__device__ __forceinline__ unsigned hdr_byte(const uint4& h, int k) {
    const unsigned w = k < 4 ? h.y : k < 8 ? h.z : h.w;
    return (w >> (8 * (k & 3))) & 0xFFu;
}
__device__ __forceinline__ void q4k_scale_min(const uint4& h, int j, float& sc, float& m) {
    if (j < 4) {
        sc = (float) (hdr_byte(h, j) & 63);
        m = (float) (hdr_byte(h, j + 4) & 63);
    } else {
        sc = (float) ((hdr_byte(h, j + 4) & 0xF) | ((hdr_byte(h, j - 4) >> 6) << 4));
        m = (float) ((hdr_byte(h, j + 4) >> 4) | ((hdr_byte(h, j) >> 6) << 4));
    }
}

// agent-scope loads for data another workgroup wrote earlier in the same launch
__device__ __forceinline__ float load_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------------------ async LDS copies
// Global -> LDS copies (global_load_lds) issued as inline assembly, so the compiler does not track them: it tracks such
// copies per wavefront, not per LDS object, and with one in flight it makes the next LDS read wait for every vector
// memory operation in flight (vmcnt(0)), which would drain weight requests issued long before.  The caller waits for
// its copies itself (vm_wait, then lds_barrier for other wavefronts' copies).  The copy is a compiler memory barrier
// as well, so values the compiler keeps in memory are read again after it: read blockDim.x and the like before a loop
// of copies.  lds: wave-uniform; lane l's bytes land at lds + BYTES l.
template <int BYTES> __device__ __forceinline__ void lds_copy_async(const void* g, const void* lds) {
    static_assert(BYTES == 4 || BYTES == 16, "4 or 16 bytes a lane");
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t) reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*) lds));
    if constexpr (BYTES == 16)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
// vmcnt(N), the other counters unwaited, as a compiler memory barrier (no memory access moves across it)
template <int N> __device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// the workgroup barrier after this wavefront's LDS operations, without the wait for vector memory that __syncthreads'
// fence adds; a compiler memory barrier
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ------------------------------------------------------------------------------------------------ warm-up
// Workgroup i of a launch runs on XCD i % 8.  A kernel warms lines for a later launch by loading one dword of each
// 128-byte line straight into LDS (no register is written, the load cannot be dropped or moved).  Measured: the lines
// are not in the L2 a kernel boundary later, but in the MALL behind it, which still serves them faster than HBM.
// warm_wait() before the wavefront ends, because the LDS it writes belongs to the workgroup.  `junk` is 256 bytes of
// LDS whose contents nobody reads.
constexpr int XCDS = 8, LINE = 128;
__device__ __forceinline__ void warm_line(const void* p, void* junk) { lds_copy_async<4>(p, junk); }
__device__ __forceinline__ void warm_wait() { vm_wait<0>(); }

// ------------------------------------------------------------------------------------------------ planar store
// Per matrix of R rows (a multiple of 32) x C columns, each plane of the store is tiled by RT rows and cut into 16-byte
// pieces: piece p of a row lies 16 RT bytes after piece p - 1, and piece p of the tile's RT rows is one contiguous run.
// Q4_K is tiled by 32 rows: a request that gives 32 consecutive rows' lanes the same piece (the matrix-core kernels, a
// lane per row) or 8 consecutive rows' 8 lanes each 8 consecutive pieces (the dot kernels) is whole 128-byte lines.
// Q8_0 is tiled by 4 rows, for its dot kernels' 16 lanes a row over 4 rows a wavefront (16 pieces x 4 rows, one
// contiguous KB); its matrix-core requests are then 64-byte halves of lines, the other half the next step's.
constexpr int ROWTILE = 32;   // rows in every type's tile count
template <int RT> __host__ __device__ __forceinline__ size_t tiled16(int row, size_t row_bytes, int piece) {
    return (size_t) (row / RT) * RT * row_bytes + (size_t) piece * (RT * 16) + (size_t) (row % RT) * 16;
}
constexpr int Q4K_RT = 32, Q80_RT = 4;
constexpr int PIECE_STRIDE = Q4K_RT * 16;   // Q4_K: bytes from one piece of a row to the next
// the K-quants (Q4_K, Q5_K): nibble plane, then (Q5_K) the fifth-bit plane, then the header plane
struct KqPlanes {
    const uint8_t* nib;   // R x C/2: a row's runs of 256 bytes (two super-blocks), 16-byte pieces in [half][group] order
    const uint8_t* qh;    // Q5_K: R x C/8: a super-block's 32 qh bytes as pieces 2 b, 2 b + 1
    const uint8_t* hdr;   // R x C/256 x 16: a row's super-block headers, one piece each
    // piece p (bytes 16 p .. 16 p + 15) of row r's nibble bytes
    __host__ __device__ __forceinline__ const uint8_t* nib16(int r, int C, int p) const { return nib + tiled16<Q4K_RT>(r, C / 2, p); }
    // piece p of row r's qh bytes (super-block p / 2, bytes 16 (p % 2) ..)
    __host__ __device__ __forceinline__ const uint8_t* qh16(int r, int C, int p) const { return qh + tiled16<Q4K_RT>(r, C / 8, p); }
    // the 16-byte header of super-block b of row r
    __host__ __device__ __forceinline__ const uint8_t* hdr16(int r, int C, int b) const { return hdr + tiled16<Q4K_RT>(r, C / 16, b); }
};
using Q4kPlanes = KqPlanes;
template <bool Q5> __host__ __device__ __forceinline__ KqPlanes kq_planes(const void* mat, int R, int C) {
    const uint8_t* p = (const uint8_t*) mat;
    const size_t nib = (size_t) R * (C / 2), qh = Q5 ? (size_t) R * (C / 8) : 0;
    return KqPlanes{p, p + nib, p + nib + qh};
}
__host__ __device__ __forceinline__ KqPlanes q4k_planes(const void* mat, int R, int C) { return kq_planes<false>(mat, R, C); }
__host__ __device__ __forceinline__ KqPlanes q5k_planes(const void* mat, int R, int C) { return kq_planes<true>(mat, R, C); }
struct Q80Planes {
    const uint8_t* q;     // R x C: a row's 512-byte runs (16 blocks), 16-byte pieces in [half][block] order
    const uint8_t* d;     // R x C/32 f16: a row's block scales, 8 a piece
    __host__ __device__ __forceinline__ const uint8_t* q16(int r, int C, int p) const { return q + tiled16<Q80_RT>(r, C, p); }
    __host__ __device__ __forceinline__ const uint8_t* d16(int r, int C, int p) const { return d + tiled16<Q80_RT>(r, C / 16, p); }
    // the f16 scale of block b of row r
    __host__ __device__ __forceinline__ const uint16_t* dof(int r, int C, int b) const {
        return reinterpret_cast<const uint16_t*>(d16(r, C, b / 8) + 2 * (b % 8));
    }
};
// Q4_0 / Q5_1 (tiled like Q8_0, by 4 rows): a nibble plane of R x C/2 (one 16-byte piece a block: value l in the low
// nibble of byte l, l + 16 in its high nibble), then Q4_0: an f16 d plane of R x C/16; Q5_1: a (d, m) plane of R x C/8
// and a qh plane of R x C/8 (4 bytes a block each)
struct NbPlanes {
    const uint8_t* q;
    const uint8_t* s;    // Q4_0: d; Q5_1: (d, m)
    const uint8_t* qh;   // Q5_1
    __host__ __device__ __forceinline__ const uint8_t* q16(int r, int C, int p) const { return q + tiled16<Q80_RT>(r, C / 2, p); }
    // Q4_0: block b's f16 d
    __host__ __device__ __forceinline__ const uint8_t* d_of(int r, int C, int b) const {
        return s + tiled16<Q80_RT>(r, C / 16, b / 8) + 2 * (b % 8);
    }
    // Q5_1: block b's (d, m) and its qh word; 4 blocks a piece
    __host__ __device__ __forceinline__ const uint8_t* dm_of(int r, int C, int b) const {
        return s + tiled16<Q80_RT>(r, C / 8, b / 4) + 4 * (b % 4);
    }
    __host__ __device__ __forceinline__ const uint8_t* qh_of(int r, int C, int b) const {
        return qh + tiled16<Q80_RT>(r, C / 8, b / 4) + 4 * (b % 4);
    }
};
template <int TYPE> __host__ __device__ __forceinline__ NbPlanes nb_planes(const void* mat, int R, int C) {
    const uint8_t* p = (const uint8_t*) mat;
    const size_t q = (size_t) R * (C / 2), s = TYPE == SFNX_Q4_0 ? (size_t) R * (C / 16) : (size_t) R * (C / 8);
    return NbPlanes{p, p + q, p + q + s};
}

__host__ __device__ __forceinline__ Q80Planes q80_planes(const void* mat, int R, int C) {
    const uint8_t* p = (const uint8_t*) mat;
    return Q80Planes{p, p + (size_t) R * C};
}

// A dense Q8_0 matrix in the reference's split layout (src/model.hpp:71-74 Q8S, filled by src/model.cpp:384-440
// q8split): int8 values [R][C] row-major and the f16 scale bits of each 32-value block [R][C / 32].  The shared expert's
// dense matrices cross the boundary in it.
struct Q8sPlanes {
    const int8_t* q;
    const uint16_t* d;
    // the 16 values of row r from column c (c % 16 == 0)
    __host__ __device__ __forceinline__ const uint8_t* q16(int r, int C, int c) const {
        return reinterpret_cast<const uint8_t*>(q) + (size_t) r * C + c;
    }
    __host__ __device__ __forceinline__ const uint16_t* dof(int r, int C, int b) const { return d + (size_t) r * (C / 32) + b; }
};

// a dense Q8_0 matrix (split layout) into the planar Q8_0 layout of one matrix at dst, on stream s (dense.hip)
size_t q8s_planar_bytes(int rows, int cols);
void q8s_to_planar(const sfnx_q8s& W, int rows, int cols, void* dst, hipStream_t s);

inline bool expert_type_ok(uint32_t type) {
    return type == SFNX_Q4_K || type == SFNX_Q5_K || type == SFNX_Q8_0 || type == SFNX_Q4_0 || type == SFNX_Q5_1;
}
constexpr const char* TYPE_MSG = "expert type must be Q4_0 (2), Q5_1 (7), Q8_0 (8), Q4_K (12) or Q5_K (13)";
__host__ __device__ constexpr bool is_kquant(uint32_t type) { return type == SFNX_Q4_K || type == SFNX_Q5_K; }
inline int block_values(uint32_t type) { return is_kquant(type) ? 256 : 32; }
// Expert e's matrix of a store (src/moe_w.cuh:9 moe_expert): base + e * sa, or, when sa is 0, the device table of
// expert pointers at `base` (the reference's DW::ep, src/model.hpp:85-86: each expert wherever it lives, a VRAM slot or
// mapped page-locked host memory).  sa is a kernel argument, so the branch is uniform.  The table's entries are read
// as global-memory pointers: a pointer loaded from memory is otherwise generic, and every load through it a flat
// load, which the compiler can only wait for with vmcnt(0) and lgkmcnt(0).
typedef const __attribute__((address_space(1))) uint8_t* global_u8_ptr;
__device__ __forceinline__ const uint8_t* expert_at(const uint8_t* base, size_t sa, int e) {
    if (sa) return base + (size_t) e * sa;
    return (const uint8_t*) reinterpret_cast<const global_u8_ptr*>(base)[e];
}
// N experts' matrices at once.  With a pointer table, every entry is requested and then waited for here, inside the
// table's branch: a table load left in flight past the branch would make the compiler wait for every earlier vector
// memory request at each later use on both sides (it cannot count a load issued on one side of a branch only).
// (global-memory pointers: the caller may pass them to statements the compiler cannot see into and still have its
// loads through them global)
template <int N> __device__ __forceinline__ void experts_at(const uint8_t* base, size_t sa, const int (&e)[N], global_u8_ptr (&m)[N]) {
    if (sa) {
#pragma unroll
        for (int i = 0; i < N; ++i) m[i] = (global_u8_ptr) base + (size_t) e[i] * sa;
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) m[i] = reinterpret_cast<const global_u8_ptr*>(base)[e[i]];
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the entries (and whatever was requested before them)
    }
}
// a store's stride as the launchers check it: sa == 0 is the pointer table, else at least one matrix
inline bool stride_ok(size_t sa, size_t matrix_bytes) { return sa == 0 || sa >= matrix_bytes; }

__host__ __device__ inline size_t row_bytes(uint32_t type, int cols) {
    switch (type) {
        case SFNX_Q4_K: return (size_t) cols / 256 * Q4K_BYTES;
        case SFNX_Q5_K: return (size_t) cols / 256 * Q5K_BYTES;
        case SFNX_Q4_0: return (size_t) cols / 32 * Q40_BYTES;
        case SFNX_Q5_1: return (size_t) cols / 32 * Q51_BYTES;
        default: return (size_t) cols / 32 * Q80_BYTES;
    }
}

}  // namespace sfnx

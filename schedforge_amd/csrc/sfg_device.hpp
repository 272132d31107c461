// sfg_device.hpp -- device-side helpers shared by the gfx950 kernels.
//
// bf16 values live in memory as uint16_t bit patterns.  Conversion from fp32 is
// round-to-nearest-even by adding 0x7FFF + lsb, the rule of the reference's
// convert_to_bf16 (src/compiler.cpp:34-43), so host-rounded inputs and
// device-rounded intermediates agree bit for bit on finite values.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sfg {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint16_t bf16_t;

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t bits = __float_as_uint(f);
    return static_cast<uint16_t>((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

// Two fp32 values -> packed bf16 pair (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// 8 bf16 held in a uint4 -> MFMA operand.
__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
    return __builtin_bit_cast(bf16x8, v);
}

// 8 int8 (two dwords) -> 8 bf16.  |q| <= 128 has at most 8 significant bits,
// so the fp32 value's low 16 bits are zero and truncation is exact: each
// byte converts in one instruction (sign-extending byte select), and one byte
// permute packs the high halves of two such floats (bytes 2, 3 of the first
// and 2, 3 of the second) into a bf16 pair.
__device__ __forceinline__ uint32_t hi16_pair(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}
__device__ __forceinline__ uint4 i8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
    uint4 r;
    const int8_t* p0 = reinterpret_cast<const int8_t*>(&lo);
    const int8_t* p1 = reinterpret_cast<const int8_t*>(&hi);
    r.x = hi16_pair(static_cast<float>(p0[0]), static_cast<float>(p0[1]));
    r.y = hi16_pair(static_cast<float>(p0[2]), static_cast<float>(p0[3]));
    r.z = hi16_pair(static_cast<float>(p1[0]), static_cast<float>(p1[1]));
    r.w = hi16_pair(static_cast<float>(p1[2]), static_cast<float>(p1[3]));
    return r;
}

// 8 fp32 -> 8 bf16 packed in a uint4.
__device__ __forceinline__ uint4 f32x8_to_bf16x8(const float* v) {
    uint4 r;
    r.x = pack_bf16x2(v[0], v[1]);
    r.y = pack_bf16x2(v[2], v[3]);
    r.z = pack_bf16x2(v[4], v[5]);
    r.w = pack_bf16x2(v[6], v[7]);
    return r;
}

// silu(v) = v / (1 + e^-v), the division as a multiply by the hardware
// reciprocal (1 ulp): the IEEE division's refinement sequence cost the GEMM
// epilogues a third of their VALU time.  Large negative v: e^-v = inf,
// reciprocal 0, result -0 (the division's limit).
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// The value lane l ^ 32 (resp. l ^ 16) holds, combined with this lane's by
// max or +, from v_permlane32_swap (v_permlane16_swap): one VALU op instead
// of a ds_bpermute round trip through LDS.  Two-operand max and sum are
// commutative, so each lane gets the same bits as f(v, shfl_xor(v, 32)).
__device__ __forceinline__ float xor32_max(float v) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// The value of lane l ^ X for X = 1, 2, 4, 8, by DPP inside 16-lane rows:
// quad_perm for 1 and 2, row_ror:8 for 8, and for 4 two moves under bank
// masks (banks 0 and 2 take lane l + 4 by row_ror:12, banks 1 and 3 lane
// l - 4 by row_ror:4).
template <int CTRL, int BANKS = 0xF>
__device__ __forceinline__ float dpp_mov(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, 0xF, BANKS, false));
}
__device__ __forceinline__ float lane_xor1(float v) { return dpp_mov<0xB1>(v, v); }
__device__ __forceinline__ float lane_xor2(float v) { return dpp_mov<0x4E>(v, v); }
__device__ __forceinline__ float lane_xor4(float v) { return dpp_mov<0x124, 0xA>(dpp_mov<0x12C, 0x5>(v, v), v); }
__device__ __forceinline__ float lane_xor8(float v) { return dpp_mov<0x128>(v, v); }

// Sum and max over the wave by the xor butterfly 32, 16, 8, 4, 2, 1 (each
// step v op partner), without LDS: the float sum has the same association,
// hence the same bits, as the same butterfly over __shfl_xor.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}
template <>
__device__ __forceinline__ float wave_sum<float>(float v) {
    v = xor32_sum(v);
    v = xor16_sum(v);
    v += lane_xor8(v);
    v += lane_xor4(v);
    v += lane_xor2(v);
    v += lane_xor1(v);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = xor32_max(v);
    v = xor16_max(v);
    v = fmaxf(v, lane_xor8(v));
    v = fmaxf(v, lane_xor4(v));
    v = fmaxf(v, lane_xor2(v));
    return fmaxf(v, lane_xor1(v));
}

// Lane `src`'s value in every lane (v_readlane_b32); src must be the same in
// every lane of the wave.
__device__ __forceinline__ float lane_bcast(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ __forceinline__ int lane_bcast(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

// v_exp_f32: 2^x.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// 16 bytes per lane from global memory into LDS at lds_block + 16 * lane
// (global_load_lds_dwordx4; lds_block is wave-uniform).  A __device__
// function, not a lambda: the builtin exists on the device side only.
__device__ __forceinline__ void lds_dma16(const uint16_t* src, uint16_t* lds_block) {
    __builtin_amdgcn_global_load_lds(src, lds_block, 16, 0, 0);
}

// The same 16-byte-per-lane LDS DMA through a buffer resource
// (buffer_load_dwordx4 ... lds): byte offset voffset from the resource's base,
// loads past its num_records bytes return zeros instead of faulting.  Unlike
// the global form, the compiler does not count it as a pending FLAT access, so
// fragment reads issued while it is in flight keep partial lgkmcnt waits.
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, uint32_t bytes) {
    // dword3 0x00020000: 32-bit data format, the raw-buffer setting of gfx9 parts
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ void lds_dma16_buf(buf_rsrc r, uint32_t voffset, uint16_t* lds_block) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)(lds_block), 16, voffset, 0, 0, 0);
}
// A DMA of BYTES (4 or 16) per lane, wave-uniform byte offset in the SGPR
// operand; the wave's 64 lanes fill 64 * BYTES contiguous LDS bytes.
template <int BYTES>
__device__ __forceinline__ void lds_dma_buf(buf_rsrc r, uint32_t voffset, uint32_t soffset,
                                            uint16_t* lds_block) {
    static_assert(BYTES == 4 || BYTES == 16, "LDS DMA moves 4 or 16 bytes per lane here");
    auto* dst = (__attribute__((address_space(3))) void*)(lds_block);
    if constexpr (BYTES == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voffset, soffset, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, voffset, soffset, 0, 0);
}
// The same load with a wave-uniform byte offset in the instruction's SGPR
// operand: a loop that advances only `soffset` issues each load without any
// per-lane address arithmetic.
__device__ __forceinline__ void lds_dma16_buf(buf_rsrc r, uint32_t voffset, uint32_t soffset,
                                              uint16_t* lds_block) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)(lds_block), 16, voffset, soffset, 0, 0);
}

__device__ __forceinline__ void wait_vmem_all() {
    // s_waitcnt vmcnt(0), other counters untouched (gfx9 encoding: expcnt 7,
    // lgkmcnt 15).  LDS DMA completes through vmcnt.
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

// s_waitcnt vmcnt(N), expcnt and lgkmcnt untouched (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmem() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// s_waitcnt vmcnt(N) lgkmcnt(0): this wave's older loads and all its LDS
// accesses are done.
template <int N>
__device__ __forceinline__ void wait_vmem_lds() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
}

// Workgroup barrier without __syncthreads()'s release fence, which would wait
// for every outstanding load (vmcnt(0)) including the LDS DMA of the stages
// still meant to be in flight.  The memory clobber keeps the compiler from
// moving LDS accesses across it; each wave has already waited for its own
// loads of the stage about to be read, and LDS is coherent inside the CU.
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_barrier" ::: "memory"); }

// s_waitcnt lgkmcnt(0), vmcnt and expcnt untouched: this wave's LDS accesses
// (reads and writes) are done.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Two fp32 -> packed bf16 pair with the hardware converter
// (v_cvt_pk_bf16_f32, round to nearest even: the same bits as pack_bf16x2 for
// finite values).
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    const f32x2v v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}

}  // namespace sfg

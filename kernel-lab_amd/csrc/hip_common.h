// Device helpers shared by the gfx950 kernels: element conversions with
// round-to-nearest-even, 16-byte vector types, and wave64 reductions built on
// DPP row operations plus lane reads.
//
// Reference counterpart: csrc/common.cuh:11-66 (Num<T>, Pack<T,N>, warp_sum,
// block_sum). The reference reduces over 32-lane warps with xor shuffles; on
// CDNA a wavefront has 64 lanes, so the reductions here work within DPP rows
// of 16 lanes and then combine the four rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace kl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- elements
// Element traits. `S` is the storage type in memory; to_f32/from_f32 are the
// exact widening and the round-to-nearest-even narrowing that PyTorch's
// `.float()` and `.to(dtype)` perform.
struct F32 {
  using S = float;
  static constexpr int kBytes = 4;
  static __device__ __forceinline__ float to_f32(S v) { return v; }
  static __device__ __forceinline__ S from_f32(float f) { return f; }
};

struct F16 {
  using S = uint16_t;
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float to_f32(S v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  }
  // v_cvt_f16_f32 rounds to nearest even in the default float mode.
  static __device__ __forceinline__ S from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};

struct BF16 {
  using S = uint16_t;
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float to_f32(S v) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(v) << 16);
  }
  // gfx950 converts with v_cvt_pk_bf16_f32, round to nearest even.
  static __device__ __forceinline__ S from_f32(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
};

// OCP FP8 E4M3 ("e4m3fn": bias 7, no infinities, NaN = S.1111.111), a storage
// format only: values are decoded before any arithmetic.
struct Fp8E4M3 {
  using S = uint8_t;
  static constexpr int kBytes = 1;
};

// Two e4m3 codes (bytes 0-1, or 2-3 when HI, of w) decoded to a packed pair of
// E (fp16 or bf16), first code in the low half. Every e4m3 value, NaN and the
// signed zeros included, is exact in both types; gfx950's conversion was
// checked against all 256 codes. The scale operand is 1: the caller applies
// its own per-head scales outside the inner loop.
template <typename E, bool HI>
__device__ __forceinline__ uint32_t fp8x2_to(uint32_t w) {
  if constexpr (std::is_same_v<E, BF16>) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
}

// Sixteen e4m3 codes (one 16-byte load) decoded to sixteen E values, codes
// 0-7 in lo and 8-15 in hi, memory order kept.
template <typename E>
__device__ __forceinline__ void fp8x16_to(u32x4 w, u32x4& lo, u32x4& hi) {
  lo = u32x4{fp8x2_to<E, false>(w[0]), fp8x2_to<E, true>(w[0]), fp8x2_to<E, false>(w[1]), fp8x2_to<E, true>(w[1])};
  hi = u32x4{fp8x2_to<E, false>(w[2]), fp8x2_to<E, true>(w[2]), fp8x2_to<E, false>(w[3]), fp8x2_to<E, true>(w[3])};
}

// Low / high 16-bit halves of a 32-bit word as floats (fp16 or bf16 storage).
template <typename E>
__device__ __forceinline__ float lo_f32(uint32_t w) {
  return E::to_f32(static_cast<uint16_t>(w & 0xffffu));
}
template <typename E>
__device__ __forceinline__ float hi_f32(uint32_t w) {
  return E::to_f32(static_cast<uint16_t>(w >> 16));
}

// Two floats rounded to 16-bit and packed, first in the low half. A
// two-element conversion is one v_cvt_pk_{f16,bf16}_f32 on gfx950 (round to
// nearest even, as from_f32); converting the halves one by one took two
// conversions, a shift and an or.
template <typename E>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (std::is_same_v<E, BF16>) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  } else if constexpr (std::is_same_v<E, F16>) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  } else {
    return static_cast<uint32_t>(E::from_f32(a)) | (static_cast<uint32_t>(E::from_f32(b)) << 16);
  }
}

// ------------------------------------------------------------------- DPP
// dpp_ctrl encodings (GCN3+ DPP): quad_perm is two bits per lane of a quad;
// row_ror:n rotates the 16 lanes of each row by n.
constexpr int kDppQuadSwap1 = 0xB1;  // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;  // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
// row_shr:n moves lane i's value to lane i + n of the same 16-lane row.
constexpr int kDppRowShr1 = 0x111;
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_read(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets its row's sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppQuadSwap1>(v);
  v += dpp<kDppQuadSwap2>(v);
  v += dpp<kDppRowRor4>(v);
  v += dpp<kDppRowRor8>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp<kDppRowRor4>(v));
  v = fmaxf(v, dpp<kDppRowRor8>(v));
  return v;
}

// Inclusive prefix sum over the wave's 64 lanes (lane i gets v[0] + ... +
// v[i]) without LDS: a Hillis-Steele scan inside each 16-lane row by DPP row
// shifts (a lane shifted in from before the row's start reads 0), then every
// row adds the totals of the rows before it, read from lanes 15, 31 and 47.
// Having no LDS instruction, it leaves the LDS/scalar-memory counter alone, so
// a scalar load issued before it stays in flight. Checked on MI355X against
// sequential sums (unit steps, lone values in lanes 0 and 63, random signed).
__device__ __forceinline__ int wave_prefix_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr1, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr2, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr4, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr8, 0xF, 0xF, true);
  const int r0 = __builtin_amdgcn_readlane(v, 15);
  const int r1 = __builtin_amdgcn_readlane(v, 31);
  const int r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = __lane_id() >> 4;
  return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// Sum over the whole wave64, returned wave-uniform. The four row sums are
// added in a fixed order, so the result does not depend on scheduling.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}

// Cross-row butterflies on gfx950's v_permlane{16,32}_swap. With both operands
// equal to v, the two results hold, in some order, v of this lane and v of
// lane ^ 16 (or lane ^ 32), so a commutative op over them is the butterfly
// step; no LDS traffic and no lane-dependent select.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<unsigned>(r[0])),
               __builtin_bit_cast(float, static_cast<unsigned>(r[1])));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<unsigned>(r[0])),
               __builtin_bit_cast(float, static_cast<unsigned>(r[1])));
}
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return __builtin_bit_cast(float, static_cast<unsigned>(r[0])) +
         __builtin_bit_cast(float, static_cast<unsigned>(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return __builtin_bit_cast(float, static_cast<unsigned>(r[0])) +
         __builtin_bit_cast(float, static_cast<unsigned>(r[1]));
}

// Raw buffer loads: a wave-uniform 128-bit resource (base address in SGPRs)
// plus a 32-bit per-lane byte offset. The address never occupies VGPRs, so
// deep software pipelines keep their loads in flight without register
// conflicts. Dword 3 selects the 32-bit data format that untyped loads need
// on the gfx9 family; num_records bounds the offsets to 2 GiB past the base.
constexpr int kBufferDword3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), 0x7fffffff,
                                           kBufferDword3);
}

// A resource covering exactly `bytes` bytes from `base`: a load at an offset
// past them returns 0 without touching memory (the hardware's range check), so
// lanes beyond the end of an array need no branch around their load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_bytes(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           kBufferDword3);
}

// A pointer that is the same in every lane, made provably wave-uniform
// (scalar registers), so a buffer resource built from it stays scalar; built
// from a per-lane value, every buffer access becomes a per-lane loop.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Cache-policy bits of the buffer instruction (gfx940+ encoding): NT marks a
// streaming access, which measured ~13% more HBM read bandwidth than the
// default policy for data read once.
constexpr int kCachePolicyNT = 2;

// Device-scope coherence (the sc1 bit): a store is written through to where
// every XCD sees it and a load does not return a line another XCD may have
// changed. It is the encoding this compiler gives relaxed agent-scope atomic
// loads and stores on gfx950, used here for plain data that workgroups on
// different XCDs exchange within one launch, without the whole-L2 write-back
// and invalidate of an agent-scope fence.
constexpr int kCachePolicyDevice = 16;

template <int POLICY = 0>
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_offset, 0, POLICY));
}

template <int POLICY = 0>
__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, byte_offset, 0, POLICY));
}

template <int POLICY = 0>
__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, byte_offset, 0, POLICY);
}

template <int POLICY = 0>
__device__ __forceinline__ void buffer_store_f32(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rsrc, byte_offset, 0, POLICY);
}

// Waits until every vector memory access this wave issued has completed
// (s_waitcnt vmcnt(0); gfx9 counts stores there too). After device-scope
// stores it orders them before a following device-scope atomic, which is
// what a release needs when no ordinary store has to be written back. The
// signal fences keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void wait_vector_memory() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt and lgkmcnt unconstrained
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Waits until at most N of this wave's vector-memory operations are in flight
// (s_waitcnt vmcnt(N); the other counters unconstrained). They complete in
// issue order, so every operation issued before the last N is done. The
// signal fences keep the compiler from moving memory accesses across it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Non-temporal load straight to LDS (gfx950 buffer_load_dwordx4 ... lds):
// lane l's 16 bytes at `byte_offset` past `base` land at dst + 16 l; lanes at
// or past `records` bytes write zeros and read no memory. `base`, `records`
// and `dst` must be wave-uniform. Issued as an asm statement: the compiler
// then tracks neither the vmcnt slot it takes nor the LDS it writes, so it
// adds no waits of its own for it (its tracking of these loads is
// conservative or absent depending on the address arithmetic), and readers
// of `dst` must wait explicitly (wait_vmcnt).
__device__ __forceinline__ void buffer_load16_lds_nt(const void* base, int records, void* dst, uint32_t byte_offset) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const i32x4 rsrc = {static_cast<int>(static_cast<uint32_t>(b)), static_cast<int>((b >> 32) & 0xffff), records,
                      kBufferDword3};
  typedef __attribute__((address_space(3))) char* lds_char;
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char)(dst)));
  asm volatile("buffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"{m0}"(lds), "v"(byte_offset), "s"(rsrc) : "memory");
}

// The 4-byte form of buffer_load16_lds_nt (default cache policy): lane l's
// dword lands at dst + 4 l.
__device__ __forceinline__ void buffer_load4_lds(const void* base, int records, void* dst, uint32_t byte_offset) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const i32x4 rsrc = {static_cast<int>(static_cast<uint32_t>(b)), static_cast<int>((b >> 32) & 0xffff), records,
                      kBufferDword3};
  typedef __attribute__((address_space(3))) char* lds_char;
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char)(dst)));
  asm volatile("buffer_load_dword %1, %2, 0 offen lds" ::"{m0}"(lds), "v"(byte_offset), "s"(rsrc) : "memory");
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16). Within each 16-lane row,
// lane i receives element (i % 4) of the 8-byte chunks addressed by lanes
// i/4, 4 + i/4, 8 + i/4 and 12 + i/4 of that row, in that order.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// Cross-row exchange (lane ^ 16, lane ^ 32) through the LDS crossbar.
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  const int lane = __lane_id();
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2,
                                                                __builtin_bit_cast(int, v)));
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// A read-only int32 table (block tables, sequence lengths) seen through the
// constant address space. A kernel that stores to global memory between its
// loads otherwise loses the proof that the table is unclobbered, and the
// compiler then fetches wave-uniform entries with vector loads whose result
// waits (s_waitcnt vmcnt) also drain every K/V load still in flight; from the
// constant space a uniform address becomes a scalar load. Only for memory no
// kernel of the launch writes.
typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
typedef const __attribute__((address_space(4))) float* const_f32_ptr;
__device__ __forceinline__ const_i32_ptr as_constant(const int32_t* p) {
  return (const_i32_ptr)(p);
}
__device__ __forceinline__ const_f32_ptr as_constant(const float* p) {
  return (const_f32_ptr)(p);
}

}  // namespace kl

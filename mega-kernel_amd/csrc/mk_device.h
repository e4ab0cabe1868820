// Device primitives for the gfx950 decode mega-kernel: bf16 unpacking, coherent (device-scope)
// loads/stores for cross-workgroup exchange, wave64 reductions and bounded spin waits.
//
// Replaces the warp32 helpers of /root/reference/config.cuh:93-179 (shuffle trees, block sums,
// silu). Everything here is written for CDNA4: 64-lane waves, DPP row operations for 16-lane
// groups, ds_bpermute to cross rows, and the gfx950 cache-policy bits (sc1 = device
// scope) for memory that other workgroups -- possibly on another XCD with its own L2 -- read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mk {

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even fp32 -> bf16 with the hardware conversion (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// ---------------------------------------------------------------------------------------------
// Memory access with explicit cache policy.
//
// On MI355X each XCD has its own L2. A plain store can sit dirty in the writer's L2; a plain
// load can hit a stale line in the reader's L1/L2. Device-scope ("sc1") stores write through to
// the memory side and device-scope loads never return a stale copy, so every buffer that one
// workgroup writes and another reads within a launch goes through these helpers.
// ---------------------------------------------------------------------------------------------
constexpr int CPOL_SC1 = 16;  // gfx940+ cache-policy bit: device (agent) scope

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ uint32_t ld_dev_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Sets status bits with a device-scope atomic OR (a vector-memory atomic of each active lane), so
// that bits other workgroups set concurrently are kept, then a release fence: every store this
// wave makes afterwards (its later exchange publishes) becomes visible only after the bit, so a
// workgroup that consumes such a publish and then reads the status word sees the bit.
__device__ __forceinline__ void raise_status(uint32_t* p, uint32_t bits) {
  __hip_atomic_fetch_or(p, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

// Global-address-space views. Pointers that come out of memory (the layer table) or through
// lambdas are generic to the compiler, and generic accesses become FLAT instructions, which count
// against the LDS counter as well as the vector-memory counter: every LDS wait would then also
// wait for all outstanding weight loads. These casts keep such accesses global.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gp(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gpw(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

// 16-byte global load (cached).
__device__ __forceinline__ uint4 ld_global16(const uint4* p) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  u4 v = *(const __attribute__((address_space(1))) u4*)p;
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Weight stream: 16 bytes, non-temporal (each weight byte is read once per token).
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  u4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u4*)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Wait until every outstanding vector-memory operation of this wave has completed (stores
// acknowledged), so a following signal cannot overtake the data it announces.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// ---------------------------------------------------------------------------------------------
// wave64 reductions (DPP inside 16-lane rows, ds_bpermute across rows)
// ---------------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// Sum over each 16-lane row; every lane of the row receives the row total.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}
// Values of the lane holding the same position in the other 16-lane row of the pair (rows 0<->1,
// 2<->3) and in the other 32-lane half, via the gfx950 lane-swap instructions (VALU, no LDS
// traffic). Each builtin returns (own, partner) in some order; these combine them symmetrically.
__device__ __forceinline__ float xsum16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xmax16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Full wave sum; every lane receives the result.
__device__ __forceinline__ float wave_sum(float v) { return xsum32(xsum16(row16_sum(v))); }

__device__ __forceinline__ unsigned xcc_id() {
  return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));  // HW_REG_XCC_ID[3:0]
}

}  // namespace mk

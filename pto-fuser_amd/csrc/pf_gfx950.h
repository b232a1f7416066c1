// gfx950-specific building blocks shared by the pipelined kernels: raw buffer descriptors and
// 16-byte buffer loads, swizzled 16-byte LDS stores, the LDS transpose read, bf16 packing and the
// bf16 MFMA, and the renormalisation threshold of the deferred state decay.
#pragma once

#include "pf_device.h"

namespace pf {

typedef short i16x4 __attribute__((ext_vector_type(4)));

// Cache-policy operand of the raw buffer builtins for a non-temporal (streaming) access.
constexpr int kCachePolicyNT = 2;

// Longest chain (tokens of one (b, h)) the entry points accept: a chain's o rows (T x 128 fp32)
// are addressed through one buffer descriptor, whose byte range and offsets are 32-bit; the limit
// keeps them below 2^31.
constexpr int kMaxChainTokens = 1 << 22;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Store of a 16-byte row vector into a Swz<RS,1> tile slot whose 8-byte halves are swapped when
// `swap` (a compile-time constant at every call): the halves change places in registers and the
// LDS store stays one conflict-free 16-byte write (two 8-byte stores would conflict).
__device__ __forceinline__ void put16(bf16* dst, const uint4& x, bool swap) {
  *reinterpret_cast<uint4*>(dst) = swap ? make_uint4(x.z, x.w, x.x, x.y) : x;
}

// Transposed 8-byte LDS read (see the header comment); p is an LDS address.
__device__ __forceinline__ bf16x4 lds_read_tr(const bf16* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(const_cast<bf16*>(p)));
  return __builtin_bit_cast(bf16x4, v);
}

__device__ __forceinline__ bf16x8 cat8(const bf16x4& lo, const bf16x4& hi) {
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ bf16x8 pack8(const floatx4& d0, const floatx4& d1) {
  return bf16x8{(bf16)d0[0], (bf16)d0[1], (bf16)d0[2], (bf16)d0[3],
                (bf16)d1[0], (bf16)d1[1], (bf16)d1[2], (bf16)d1[3]};
}

__device__ __forceinline__ floatx4 mfma_bf16(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Renormalisation threshold of the deferred state decay (log of the smallest factor kept).
constexpr float kLogFactorFloor = -60.f;

}  // namespace pf

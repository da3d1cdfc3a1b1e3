// Shared device helpers for the gfx950 RecoverSSM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn_recoverssm_hip.h"

namespace gdn {

// ----------------------------------------------------------------------------
// Element conversions. bf16 <-> f32 are bit operations (round-to-nearest-even on
// the way down, NaN kept quiet); f16 uses the hardware conversion.
// ----------------------------------------------------------------------------
struct bf16 {
  uint16_t bits;
};
using f16 = _Float16;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return __uint_as_float(uint32_t(x.bits) << 16); }
__device__ __forceinline__ float to_f32(f16 x) { return float(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16{uint16_t((u >> 16) | 0x0040u)};
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16{uint16_t(u >> 16)};
}
// The conversion starts from the rounded FP32 value: left to itself the
// compiler folds a multiply-add that produced x into the conversion (one
// mixed-precision FMA rounded once, straight to f16), which differs in the last
// bit now and then from computing in FP32 and then storing in f16.
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) {
  asm volatile("" : "+v"(x));
  return f16(x);
}

// Load one element of a runtime-typed tensor as f32 (activations, gates).
__device__ __forceinline__ float load_as_f32(const void *p, int64_t i, int dt) {
  switch (dt) {
    case GDN_DT_BF16: return to_f32(static_cast<const bf16 *>(p)[i]);
    case GDN_DT_F16: return to_f32(static_cast<const f16 *>(p)[i]);
    default: return static_cast<const float *>(p)[i];
  }
}

// Wave-uniform words gathered by one vector load: every lane reads the 32-bit
// word at its own address and readlane hands lane i's word to the whole wave.
// A wave's offsets, slot, gates and pending plan are read this way, a few
// words per lane-indexed load and one wait each, instead of one load and one
// wait per word: as separate loads the compiler issued each only after the
// previous one returned, and three serial round trips under the load of the
// other waves' state streams took a third of a wave's life before its first
// state load could issue.
// Through the global address space: a flat load would also count against the
// LDS / scalar counter, and every LDS wait would then wait for it.
__device__ __forceinline__ uint32_t lane_word(uintptr_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(1))) uint32_t *>(addr);
}
__device__ __forceinline__ uint32_t word_of(uint32_t w, int i) { return uint32_t(__builtin_amdgcn_readlane(int(w), i)); }
// int32 or int64 element from its low and high words (for int32 the high
// word is a second read of the low one).
__device__ __forceinline__ int64_t index_of(uint32_t lo, uint32_t hi, bool i64) {
  return i64 ? int64_t((uint64_t(hi) << 32) | lo) : int64_t(int32_t(lo));
}
__device__ __forceinline__ uintptr_t elem_addr(const void *p, int64_t i, bool i64) {
  return reinterpret_cast<uintptr_t>(p) + uintptr_t(i) * (i64 ? 8u : 4u);
}

// Kernel arguments are read through the scalar cache, each where the compiler
// first needs its value, so a wave on a cold cache met one miss after another
// (the fused plan + fold launch's arguments span 28 lines of 64 bytes).
// Reading one word of every line first, in one batch, makes that a single
// round trip (the B=64 fold 1 us shorter). Reads stay inside the BYTES the
// arguments occupy; call it first in the kernel.
template <int BYTES>
__device__ __forceinline__ void warm_kernel_args() {
  static_assert(BYTES <= 32 * 64, "argument block larger than the lines touched below");
  const auto *k = (const __attribute__((address_space(4))) uint32_t *)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t w[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) w[i] = i * 64 < BYTES ? k[i * 16] : 0u;
  // One consumer of every word: the reads are issued together and waited for once.
  asm volatile("" ::"s"(w[0]), "s"(w[1]), "s"(w[2]), "s"(w[3]), "s"(w[4]), "s"(w[5]), "s"(w[6]), "s"(w[7]),
               "s"(w[8]), "s"(w[9]), "s"(w[10]), "s"(w[11]), "s"(w[12]), "s"(w[13]), "s"(w[14]), "s"(w[15]),
               "s"(w[16]), "s"(w[17]), "s"(w[18]), "s"(w[19]), "s"(w[20]), "s"(w[21]), "s"(w[22]), "s"(w[23]),
               "s"(w[24]), "s"(w[25]), "s"(w[26]), "s"(w[27]), "s"(w[28]), "s"(w[29]), "s"(w[30]), "s"(w[31]));
}

// Division by a runtime divisor d in [1, 2^16] of a dividend x < 2^16 as one
// multiply-high: with m = floor(2^32 / d) + 1, m * d = 2^32 + e, 0 < e <= d,
// so x * m / 2^32 = x / d + x * e / (d * 2^32) and the added term stays below
// 1 / d (x * e < 2^32): the floor is exact. d = 1 (m would need 33 bits) is
// coded as m = 0. A runtime division is otherwise about 15 vector
// instructions per use.
__host__ __device__ inline uint32_t div16_magic(uint32_t d) {
  return d <= 1 ? 0u : uint32_t((uint64_t(1) << 32) / d + 1);
}
__device__ __forceinline__ uint32_t div16(uint32_t x, uint32_t m) {
  const uint32_t q = __umulhi(x, m);
  return m == 0 ? x : q;  // a select: a branch here splits the caller's code paths
}

// Load one element of a runtime-typed integer tensor as int64.
__device__ __forceinline__ int64_t load_index(const void *p, int64_t i, int dt) {
  return dt == GDN_DT_I64 ? static_cast<const int64_t *>(p)[i] : int64_t(static_cast<const int32_t *>(p)[i]);
}

// load_index through the constant address space, for tables no kernel writes
// while it reads them (block tables): at a uniform address it becomes a scalar
// load, counted apart from the vector loads in flight. Read as a global
// pointer inside a kernel that also stores, it becomes a vector load, and
// waiting for it waits for every vector load issued before it.
__device__ __forceinline__ int64_t load_index_ro(const void *p, int64_t i, int dt) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  if (dt == GDN_DT_I64) return reinterpret_cast<const __attribute__((address_space(4))) int64_t *>(a)[i];
  return int64_t(reinterpret_cast<const __attribute__((address_space(4))) int32_t *>(a)[i]);
}

__device__ __forceinline__ void store_from_f32(void *p, int64_t i, int dt, float x) {
  switch (dt) {
    case GDN_DT_BF16: static_cast<bf16 *>(p)[i] = from_f32<bf16>(x); break;
    case GDN_DT_F16: static_cast<f16 *>(p)[i] = from_f32<f16>(x); break;
    default: static_cast<float *>(p)[i] = x; break;
  }
}

// Elements per 16-byte chunk of state storage.
template <typename T>
struct Chunk {
  static constexpr int E = 16 / int(sizeof(T));
};

// Unpack one 16-byte chunk into E floats.
template <typename T>
__device__ __forceinline__ void unpack16(const uint4 &raw, float *out);
template <>
__device__ __forceinline__ void unpack16<float>(const uint4 &raw, float *out) {
  out[0] = __uint_as_float(raw.x);
  out[1] = __uint_as_float(raw.y);
  out[2] = __uint_as_float(raw.z);
  out[3] = __uint_as_float(raw.w);
}
template <>
__device__ __forceinline__ void unpack16<bf16>(const uint4 &raw, float *out) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void unpack16<f16>(const uint4 &raw, float *out) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = float(__builtin_bit_cast(f16, uint16_t(w[i] & 0xffffu)));
    out[2 * i + 1] = float(__builtin_bit_cast(f16, uint16_t(w[i] >> 16)));
  }
}

template <typename T>
__device__ __forceinline__ uint4 pack16(const float *in);
template <>
__device__ __forceinline__ uint4 pack16<float>(const float *in) {
  return make_uint4(__float_as_uint(in[0]), __float_as_uint(in[1]), __float_as_uint(in[2]), __float_as_uint(in[3]));
}
template <>
__device__ __forceinline__ uint4 pack16<bf16>(const float *in) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = uint32_t(from_f32<bf16>(in[2 * i]).bits) | (uint32_t(from_f32<bf16>(in[2 * i + 1]).bits) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}
template <>
__device__ __forceinline__ uint4 pack16<f16>(const float *in) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = uint32_t(__builtin_bit_cast(uint16_t, from_f32<f16>(in[2 * i]))) |
           (uint32_t(__builtin_bit_cast(uint16_t, from_f32<f16>(in[2 * i + 1]))) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ----------------------------------------------------------------------------
// 128-bit buffer store followed by wait states that keep its data registers
// untouched while the store reads them. With a register soffset the
// compiler's hazard model lets the next VALU instruction follow such a store
// at once, and on MI355X that has put a wrong first data dword into memory
// for some lanes (the value that next instruction read: the FP32 element the
// f16 conversion after the store was reading). The asm names the data
// registers, so no instruction that rewrites them moves above the wait, and
// its memory clobber keeps it behind the store.
// ----------------------------------------------------------------------------
#ifndef GDN_STORE_DATA_WAIT
#define GDN_STORE_DATA_WAIT 4
#endif
typedef unsigned gdn_u32x4 __attribute__((ext_vector_type(4)));
template <int AUX>
__device__ __forceinline__ void store_b128_settled(gdn_u32x4 v, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, AUX);
  asm volatile("s_nop %1" ::"v"(v), "n"(GDN_STORE_DATA_WAIT) : "memory");
}

// ----------------------------------------------------------------------------
// Cross-lane sums inside aligned groups of 8 lanes with DPP (no LDS traffic):
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], then row_half_mirror, which pairs
// lane i with lane 7-i of the same 8-lane half-row.
// ----------------------------------------------------------------------------
__device__ __forceinline__ float dpp_sum8(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));
  return x;
}

// Thread-local error message set by the host entry points.
void set_error(const char *fmt, ...);

// Bytes of state a verify launch reads with ordinary loads, from the end of
// its batch (gdn_recoverssm_set_state_cache_retain).
int64_t state_cache_retain();

}  // namespace gdn

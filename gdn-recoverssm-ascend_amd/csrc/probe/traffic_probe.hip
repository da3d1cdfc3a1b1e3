// Traffic probes: synthetic kernels that move the bytes of a verify or a fold
// launch in the same access pattern, with no arithmetic, to measure what the
// memory system sustains for that pattern on this GPU. bench.py runs them on
// the workload's own state tiles beside the kernels' own times. They are
// measurement tools, not part of the verify / commit path, and live in a
// library of their own (libgdn_recoverssm_probe.so).
//
// Tiles are 64 KiB (page, value head) state tiles of 128 rows x 512 bytes
// (K = V = 128, FP32), addressed by byte offsets from a base pointer.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kTileBytes = 65536;
constexpr int kRowBytes = 512;
constexpr int kNT = 2;  // buffer cache policy: non-temporal (the fold's)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const char *p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(p), 0, bytes, 0x00020000);
}

// The verify's traffic: one wave per tile; `small_dw` dwords read from a
// region two consecutive waves share (q and k are shared by the two value
// heads of a key head); the tile streamed as eight 16-row blocks, two blocks
// in flight; `write_dw` dwords written per wave, half after each 64-row half
// tile, as the verify stores its outputs and records. Tiles w < nt_tiles read
// row runs with non-temporal loads (lane l, load j: row 4 (j % 4) + l / 16,
// 16-byte chunk 16 (j / 4) + l % 16 of the block: 4 rows x 256 bytes), the
// rest the matrix-core operand layout with ordinary loads (lane (r = l % 16,
// s = l / 16) reads the 16-byte chunks 4j + s of row r), as the verify's two
// bodies do.
template <bool NT>
__device__ __forceinline__ float verify_twin_tile(__amdgpu_buffer_rsrc_t r, __amdgpu_buffer_rsrc_t wr, int lane,
                                                  int write_dw, float acc) {
  constexpr int pol = NT ? kNT : 0;
  int voff[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    voff[j] = NT ? ((j & 3) * 4 + (lane >> 4)) * kRowBytes + ((j >> 2) * 16 + (lane & 15)) * 16
                 : (lane & 15) * kRowBytes + (4 * j + (lane >> 4)) * 16;
  u32x4 a[8], b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = __builtin_amdgcn_raw_buffer_load_b128(r, voff[j], 0, pol);
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = __builtin_amdgcn_raw_buffer_load_b128(r, voff[j], 16 * kRowBytes, pol);
  const int per_half = write_dw / 2;
#pragma unroll
  for (int blk = 0; blk < 8; blk += 2) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += __uint_as_float(a[j][0] ^ a[j][3]);
    if (blk + 2 < 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = __builtin_amdgcn_raw_buffer_load_b128(r, voff[j], (blk + 2) * 16 * kRowBytes, pol);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += __uint_as_float(b[j][0] ^ b[j][3]);
    if (blk + 3 < 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = __builtin_amdgcn_raw_buffer_load_b128(r, voff[j], (blk + 3) * 16 * kRowBytes, pol);
    }
    if (blk == 2 || blk == 6) {
      const int base = blk == 2 ? 0 : per_half;
      const int n = blk == 2 ? per_half : write_dw - per_half;
      for (int i = lane; i < n; i += 64)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc + float(i)), wr, (base + i) * 4, 0, 0);
    }
  }
  return acc;
}

__global__ __launch_bounds__(64) void verify_twin(const char *__restrict__ state, const int64_t *__restrict__ tiles,
                                                  const float *__restrict__ small, int small_dw,
                                                  float *__restrict__ wbuf, int write_dw, float *__restrict__ sink,
                                                  int nt_tiles) {
  const int64_t w = blockIdx.x;
  const int lane = threadIdx.x;
  const __amdgpu_buffer_rsrc_t r = tile_rsrc(state + tiles[w], kTileBytes);
  float acc = 0.0f;
  const float *sp = small + (w / 2) * int64_t(small_dw);
  for (int i = lane; i < small_dw; i += 64) acc += sp[i];
  const __amdgpu_buffer_rsrc_t wr = tile_rsrc(reinterpret_cast<const char *>(wbuf + w * int64_t(write_dw)), write_dw * 4);
  if (w < nt_tiles)
    acc = verify_twin_tile<true>(r, wr, lane, write_dw, acc);
  else
    acc = verify_twin_tile<false>(r, wr, lane, write_dw, acc);
  // Every lane's loads feed the stored value (a store by lane 0 alone would
  // let the compiler drop the other lanes' loads); the test never holds.
  if (__float_as_uint(acc) == 0x7f800001u) sink[w] = acc;
}

// The fold's traffic: one 256-thread workgroup per tile; each thread reads
// its sixteen 16-byte chunks of the source tile (thread t, pass i: bytes
// t * 16 + i * 4096), all before the first store, then writes them to the
// boundary tile (when given) and to the final tile; loads and stores
// non-temporal, as the fold's.
__global__ __launch_bounds__(256) void fold_twin(const char *__restrict__ src, char *__restrict__ dst,
                                                 const int64_t *__restrict__ src_off,
                                                 const int64_t *__restrict__ dst_off,
                                                 const int64_t *__restrict__ dst2_off) {
  const int64_t w = blockIdx.x;
  const int t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rs = tile_rsrc(src + src_off[w], kTileBytes);
  const __amdgpu_buffer_rsrc_t rd = tile_rsrc(dst + dst_off[w], kTileBytes);
  const int64_t b2 = dst2_off[w];
  const __amdgpu_buffer_rsrc_t rb = tile_rsrc(dst + (b2 >= 0 ? b2 : dst_off[w]), b2 >= 0 ? kTileBytes : 0);
  u32x4 x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, t * 16, i * 4096, kNT);
#pragma unroll
  for (int i = 0; i < 16; ++i) __builtin_amdgcn_raw_buffer_store_b128(x[i], rb, t * 16, i * 4096, kNT);
#pragma unroll
  for (int i = 0; i < 16; ++i) __builtin_amdgcn_raw_buffer_store_b128(x[i], rd, t * 16, i * 4096, kNT);
}

}  // namespace

// Returns 0, or 1 when the arguments are out of range (nothing launched), or
// 3 when the launch fails. Offsets are tile byte offsets from the bases;
// write_dw bytes fit a 32-bit buffer extent.
extern "C" int gdn_probe_verify_twin(const void *state, const int64_t *tile_offsets, int64_t n_tiles,
                                     const float *small, int64_t small_dw, float *wbuf, int64_t write_dw,
                                     float *sink, int64_t nt_tiles, void *stream) {
  if (!state || !tile_offsets || !sink || n_tiles <= 0 || n_tiles > 0x7fffffffLL || small_dw < 0 ||
      small_dw > (1 << 20) || write_dw < 0 || write_dw > (1 << 20) || (small_dw && !small) || (write_dw && !wbuf))
    return 1;
  hipLaunchKernelGGL(verify_twin, dim3(unsigned(n_tiles)), dim3(64), 0, static_cast<hipStream_t>(stream),
                     static_cast<const char *>(state), tile_offsets, small, int(small_dw), wbuf, int(write_dw), sink,
                     int(nt_tiles < 0 ? 0 : nt_tiles > n_tiles ? n_tiles : nt_tiles));
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int gdn_probe_fold_twin(const void *src, void *dst, const int64_t *src_off, const int64_t *dst_off,
                                   const int64_t *dst2_off, int64_t n_tiles, void *stream) {
  if (!src || !dst || !src_off || !dst_off || !dst2_off || n_tiles <= 0 || n_tiles > 0x7fffffffLL) return 1;
  hipLaunchKernelGGL(fold_twin, dim3(unsigned(n_tiles)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const char *>(src), static_cast<char *>(dst), src_off, dst_off, dst2_off);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

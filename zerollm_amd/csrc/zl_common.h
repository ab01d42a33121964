// Shared definitions of the zerollm MI355X library: ggml type ids, the repacked weight layout, error handling and
// small device helpers. Target: gfx950 (CDNA4), wave64.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdexcept>
#include <string>

#include "zerollm_hip.h"  // status codes (ZL_OK, ZL_ERR_*)

namespace zl {

// ggml tensor type ids (zerollm src/gguf/types.js:10-15)
enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};


#define ZL_HIP(x)                                                                                 \
  do {                                                                                            \
    hipError_t e_ = (x);                                                                          \
    if (e_ != hipSuccess) throw ::zl::Error(ZL_ERR_HIP, std::string(#x) + ": " + hipGetErrorString(e_)); \
  } while (0)

#define ZL_REQUIRE(cond, code, msg)               \
  do {                                            \
    if (!(cond)) throw ::zl::Error((code), (msg)); \
  } while (0)

// ---------------------------------------------------------------------------------------------- repacked weights
// Every quantised matrix is stored as planes of 64-value "slabs" (cols padded to a multiple of 64 with zero blocks),
// rows grouped in tiles of 64 (rows padded to a multiple of 64 with zeros). Within a tile the planes are slab-major:
// element (row r, slab s) has tile-slab index ts = (r / 64) * nslab + s and lane l = r % 64, and the 64 rows of one
// tile-slab are contiguous, so a wave whose lane l works on row 64T + l reads one contiguous piece per plane per slab.
//   qs  packed low bits, QB bytes per (row, slab), stored as QB/16 parts of 16 bytes: part p of (r, s) at
//       ((ts * QB/16 + p) * 64 + l) * 16 (each 16-byte load of a wave covers 1 KB without gaps).
//       Q8_0 QB 64 (int8), Q4_0/Q5_0/Q4_K/Q5_K 32 (byte j: low nibble = value j, high nibble = value j+32),
//       Q6_K 32 (same nibble layout, the low 4 of 6 bits)
//   qx  extra high bits at (ts * 64 + l) * QX: Q5_0/Q5_K QX 8 (bit j of word w = 5th bit of value 32w+j),
//       Q6_K QX 16 (byte j: bits 2i..2i+1 = top 2 bits of value j + 16i)
//   sc  4 bytes at (ts * 64 + l) * 4: Q4_K/Q5_K scale codes of the two 32-value sub-blocks, then their min codes;
//       Q6_K the four int8 16-value group scales
//   dd  f16 scales: Q8_0/Q4_0/Q5_0 two per (row, slab) at u16 index (ts * 64 + l) * 2 + h (h = 32-value block);
//       Q4_K/Q5_K (d, dmin) per 256-value super-block at u16 index ((r/64 * nsb + s/4) * 64 + l) * 2 + {0, 1};
//       Q6_K d per super-block at u16 index (r/64 * nsb + s/4) * 64 + l  (nsb = nslab / 4)
// A view of rows [64i, 64i + n) is an offset into every plane. F32/F16/BF16 matrices keep row-major values in qs.
struct DevMat {
  int type = -1, rows = 0, cols = 0, nslab = 0;
  uint8_t *qs = nullptr, *qx = nullptr, *sc = nullptr;
  uint16_t *dd = nullptr;
  uint8_t *fq = nullptr;  // Q4_K: the 4-bit plane again, in matrix-core operand order (same size as qs)
};

__host__ __device__ inline int qs_bytes(int t) { return t == T_Q8_0 ? 64 : 32; }
__host__ __device__ inline int qx_bytes(int t) { return (t == T_Q5_0 || t == T_Q5_K) ? 8 : t == T_Q6_K ? 16 : 0; }
__host__ __device__ inline int sc_bytes(int t) { return (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K) ? 4 : 0; }
__host__ __device__ inline bool is_quant(int t) { return t == T_Q8_0 || t == T_Q4_0 || t == T_Q5_0 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }
__host__ __device__ inline bool is_kquant(int t) { return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }
__host__ __device__ inline int tiles_of(int rows) { return (rows + 63) / 64; }
// u16 entries of the dd plane per 64-row tile
__host__ __device__ inline long dd_per_tile(int t, int nslab) {
  return (t == T_Q4_K || t == T_Q5_K) ? (long)(nslab / 4) * 128 : t == T_Q6_K ? (long)(nslab / 4) * 64 : (long)nslab * 128;
}

// Byte / u16 offsets of element (r, s) in the tiled planes (device side; the host uses the same formulas).
__host__ __device__ inline long tile_slab(int r, int s, int nslab) { return (long)(r >> 6) * nslab + s; }
__host__ __device__ inline long qs_off(int t, int r, int s, int nslab, int j) {  // byte j of the (r, s) slab's qs
  const int qp = t == T_Q8_0 ? 4 : 2;
  return ((tile_slab(r, s, nslab) * qp + (j >> 4)) * 64 + (r & 63)) * 16 + (j & 15);
}
__host__ __device__ inline long qx_off(int t, int r, int s, int nslab, int j) {
  return (tile_slab(r, s, nslab) * 64 + (r & 63)) * ((t == T_Q6_K) ? 16 : 8) + j;
}
__host__ __device__ inline long sc_off(int r, int s, int nslab, int j) { return (tile_slab(r, s, nslab) * 64 + (r & 63)) * 4 + j; }
__host__ __device__ inline long dd_off(int t, int r, int s, int nslab, int k) {  // k: 32-block half (per-slab types) or d/dmin
  if (t == T_Q4_K || t == T_Q5_K) return (((long)(r >> 6) * (nslab >> 2) + (s >> 2)) * 64 + (r & 63)) * 2 + k;
  if (t == T_Q6_K) return ((long)(r >> 6) * (nslab >> 2) + (s >> 2)) * 64 + (r & 63);
  return (tile_slab(r, s, nslab) * 64 + (r & 63)) * 2 + k;
}

// ---------------------------------------------------------------------------------------------- device helpers
__device__ inline float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ inline uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

__device__ inline int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// ---- cross-lane reductions over aligned groups of `width` lanes (a power of two <= 64); every lane of a group ends
// with the group's result. Steps pair lanes like an xor butterfly (1, 2, 4, 8, 16, 32): within a quad by DPP
// quad_perm, then DPP row_half_mirror / row_mirror (the partner lies in the other half of the 8- / 16-lane group, whose
// lanes all hold the same partial by then, so each step adds exactly what the xor butterfly adds), then ds_swizzle
// (xor 16) and a lane permute (xor 32). DPP moves cost no LDS round trip.
template <int CTRL>
__device__ inline int dpp_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }

template <int CTRL, typename T>
__device__ inline T dpp_move(T v) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, dpp_i32<CTRL>(__builtin_bit_cast(int, v)));
  } else {
    static_assert(sizeof(T) == 8, "32- or 64-bit lanes");
    const long long x = __builtin_bit_cast(long long, v);
    const int lo = dpp_i32<CTRL>((int)x), hi = dpp_i32<CTRL>((int)(x >> 32));
    return __builtin_bit_cast(T, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
  }
}

template <typename T>
__device__ inline T swizzle_xor16(T v) {
  constexpr int pat = (0x10 << 10) | 0x1F;  // bitmask mode: and 0x1F, or 0, xor 0x10 (within 32 lanes)
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), pat));
  } else {
    const long long x = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_ds_swizzle((int)x, pat), hi = __builtin_amdgcn_ds_swizzle((int)(x >> 32), pat);
    return __builtin_bit_cast(T, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
  }
}

template <typename T, typename Op>
__device__ inline T group_reduce(T v, int width, Op op) {
  if (width > 1) v = op(v, dpp_move<0xB1>(v));   // quad_perm [1,0,3,2]: xor 1
  if (width > 2) v = op(v, dpp_move<0x4E>(v));   // quad_perm [2,3,0,1]: xor 2
  if (width > 4) v = op(v, dpp_move<0x141>(v));  // row_half_mirror: the other quad of the 8-lane group
  if (width > 8) v = op(v, dpp_move<0x140>(v));  // row_mirror: the other 8 lanes of the row
  if (width > 16) v = op(v, swizzle_xor16(v));
  if (width > 32) v = op(v, __shfl_xor(v, 32, 64));
  return v;
}

// Uniform values (kernel arguments) needed right after a kernel's first branches: an empty asm that reads each in
// scalar registers at this point, so the compiler issues their argument loads together with the first ones instead
// of in later rounds behind the branches (each round of argument loads waits out a memory latency).
template <typename T>
__device__ __forceinline__ void pin_arg(const T &v) {
  asm volatile("" ::"s"(v));
}
template <typename... T>
__device__ __forceinline__ void pin_args(const T &...v) {
  (pin_arg(v), ...);
}

template <typename T>
__device__ inline T wave_sum_xor(T v, int width) {
  return group_reduce(v, width, [](T a, T b) { return a + b; });
}

__device__ inline float group_fmax(float v, int width) {
  return group_reduce(v, width, [](float a, float b) { return fmaxf(a, b); });
}

// Order-preserving key of a float (larger float -> larger key); -0 is folded onto +0 so that equal values have equal keys.
__device__ inline uint32_t fkey(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float keyf(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

}  // namespace zl

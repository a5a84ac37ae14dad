// Shared device helpers for the SimSD MI355X (gfx950) kernels.
//
// Everything here is CDNA4-specific: wave64, v_mfma_f32_16x16x32_{bf16,f16} and
// v_mfma_f32_16x16x4_f32 operand layouts, 128-bit global loads.
//
// MFMA 16x16 operand layout used throughout (one wave = 64 lanes):
//   lane l, group g = l / 16, r = l % 16
//   A operand (16 rows x KS k):  row r, k-chunk g  (16 bytes per lane)
//   B operand (KS k x 16 cols):  col r, k-chunk g  (16 bytes per lane)
//   C result (16 x 16 fp32):     lane l holds C[4*g + j][r], j = 0..3
// The kernels feed a weight row as the A operand (rows = output features) and an
// activation row as the B operand (cols = tokens), so each lane streams 16
// contiguous bytes of one weight row per MFMA k-step.  Which physical k a lane's
// chunk maps to is free as long as A and B agree, so one k-step consumes 64
// contiguous bytes of every row it touches, whatever the element type:
//   bf16/f16: 8 elements per lane, KS = 32, one 16x16x32 MFMA per step
//   f32:      4 elements per lane, KS = 16, four 16x16x4 MFMAs per step
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SIMSD_DEV __device__ __forceinline__

namespace simsd {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

enum : int { kBF16 = 0, kF16 = 1, kF32 = 2 };

constexpr int kWave = 64;
constexpr int kStepBytes = 64;   // bytes of one row consumed per MFMA k-step
constexpr int kLaneBytes = 16;   // bytes of one row held by one lane per k-step

template <int DT> struct DTypeInfo;
template <> struct DTypeInfo<kBF16> { static constexpr int kSize = 2; };
template <> struct DTypeInfo<kF16> { static constexpr int kSize = 2; };
template <> struct DTypeInfo<kF32> { static constexpr int kSize = 4; };

// ---------------------------------------------------------------- conversions
SIMSD_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even fp32 -> bf16, NaN kept quiet (same rule as torch's
// c10::BFloat16 constructor).
SIMSD_DEV uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int DT> SIMSD_DEV float load_elem(const char* base, int64_t idx);
template <> SIMSD_DEV float load_elem<kBF16>(const char* base, int64_t idx) {
  return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
}
template <> SIMSD_DEV float load_elem<kF16>(const char* base, int64_t idx) {
  return (float)reinterpret_cast<const _Float16*>(base)[idx];
}
template <> SIMSD_DEV float load_elem<kF32>(const char* base, int64_t idx) {
  return reinterpret_cast<const float*>(base)[idx];
}

template <int DT> SIMSD_DEV void store_elem(char* base, int64_t idx, float v);
template <> SIMSD_DEV void store_elem<kBF16>(char* base, int64_t idx, float v) {
  reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16_bits(v);
}
template <> SIMSD_DEV void store_elem<kF16>(char* base, int64_t idx, float v) {
  reinterpret_cast<_Float16*>(base)[idx] = (_Float16)v;
}
template <> SIMSD_DEV void store_elem<kF32>(char* base, int64_t idx, float v) {
  reinterpret_cast<float*>(base)[idx] = v;
}

// Round a float to the storage precision of DT and back (models torch's
// "compute in fp32, store in x.dtype" for elementwise ops).
template <int DT> SIMSD_DEV float round_to(float v);
template <> SIMSD_DEV float round_to<kBF16>(float v) {
  return bf16_bits_to_f32(f32_to_bf16_bits(v));
}
template <> SIMSD_DEV float round_to<kF16>(float v) { return (float)(_Float16)v; }
template <> SIMSD_DEV float round_to<kF32>(float v) { return v; }

// ---------------------------------------------------------------- MFMA k-step
template <int DT> struct Mfma;
template <> struct Mfma<kBF16> {
  static SIMSD_DEV f32x4_t step(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<kF16> {
  static SIMSD_DEV f32x4_t step(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<kF32> {
  // Four 16x16x4 MFMAs; in the j-th one lane group g supplies element j of its
  // 4-element chunk, identically for A and B, so every k is summed exactly once.
  static SIMSD_DEV f32x4_t step(u32x4_t a, u32x4_t b, f32x4_t c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
    return c;
  }
};

SIMSD_DEV u32x4_t zero4() { return u32x4_t{0u, 0u, 0u, 0u}; }

SIMSD_DEV u32x4_t load16(const char* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// ------------------------------------------------- fast accumulate (16 B loads)
// Rows are byte pointers to the START of a row; every row must be 16-byte
// aligned and its length Kb (bytes) a multiple of 16.  A rows are always valid
// (callers clamp out-of-range rows onto a real row and discard the result);
// a null B row contributes zeros.  Steps [s0, s1) of 64 bytes are summed.
template <int RB, int CB, int U>
SIMSD_DEV void load_batch(u32x4_t (&A)[U][RB], u32x4_t (&B)[U][CB],
                          const char* const (&arow)[RB], const char* const (&brow)[CB],
                          int s, int s1, int lane_off, int64_t Kb) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t off = (int64_t)(s + u) * kStepBytes + lane_off;
    const bool ok = (s + u < s1) && (off < Kb);
    const int64_t offc = ok ? off : 0;   // row start is always readable
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const u32x4_t v = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(arow[rb] + offc));
      A[u][rb] = ok ? v : zero4();
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      u32x4_t v = zero4();
      if (brow[cb] != nullptr && ok) v = load16(brow[cb] + off);
      B[u][cb] = v;
    }
  }
}

template <int DT, int RB, int CB, int U>
SIMSD_DEV void mfma_batch(const u32x4_t (&A)[U][RB], const u32x4_t (&B)[U][CB],
                          f32x4_t (&acc)[RB][CB]) {
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        acc[rb][cb] = Mfma<DT>::step(A[u][rb], B[u][cb], acc[rb][cb]);
}

// Double-buffered: the loads of batch i+1 are in flight while batch i feeds
// the MFMAs.
template <int DT, int RB, int CB, int U>
SIMSD_DEV void accum_fast(const char* const (&arow)[RB], const char* const (&brow)[CB],
                          int s0, int s1, int lane_off, int64_t Kb, f32x4_t (&acc)[RB][CB]) {
  if (s0 >= s1) return;
  u32x4_t A0[U][RB], B0[U][CB], A1[U][RB], B1[U][CB];
  int s = s0;
  load_batch<RB, CB, U>(A0, B0, arow, brow, s, s1, lane_off, Kb);
  while (true) {
    if (s + U >= s1) { mfma_batch<DT, RB, CB, U>(A0, B0, acc); break; }
    load_batch<RB, CB, U>(A1, B1, arow, brow, s + U, s1, lane_off, Kb);
    mfma_batch<DT, RB, CB, U>(A0, B0, acc);
    s += U;
    if (s + U >= s1) { mfma_batch<DT, RB, CB, U>(A1, B1, acc); break; }
    load_batch<RB, CB, U>(A0, B0, arow, brow, s + U, s1, lane_off, Kb);
    mfma_batch<DT, RB, CB, U>(A1, B1, acc);
    s += U;
  }
}

// ------------------------------------------------ generic accumulate (strided)
// Element-wise gathers for views the 16-byte path cannot take (K-strided,
// misaligned or odd-length rows).  Correct for any stride; slow by design.
template <int DT>
SIMSD_DEV u32x4_t gather16(const char* row, int64_t stride_k_bytes, int64_t k0, int64_t K) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (ES == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k = k0 + j;
      if (k < K) w[j] = *reinterpret_cast<const uint32_t*>(row + k * stride_k_bytes);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = k0 + j;
      if (k < K) {
        const uint32_t h = *reinterpret_cast<const uint16_t*>(row + k * stride_k_bytes);
        w[j >> 1] |= h << (16 * (j & 1));
      }
    }
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

template <int DT, int RB, int CB>
SIMSD_DEV void accum_generic(const char* const (&arow)[RB], int64_t a_sk_bytes,
                             const char* const (&brow)[CB], int64_t b_sk_bytes,
                             int s0, int s1, int g, int64_t K, f32x4_t (&acc)[RB][CB]) {
  constexpr int VEC = kLaneBytes / DTypeInfo<DT>::kSize;
  for (int s = s0; s < s1; ++s) {
    const int64_t k0 = (int64_t)s * (4 * VEC) + g * VEC;
    u32x4_t A[RB], B[CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) A[rb] = gather16<DT>(arow[rb], a_sk_bytes, k0, K);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
      B[cb] = brow[cb] != nullptr ? gather16<DT>(brow[cb], b_sk_bytes, k0, K) : zero4();
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = Mfma<DT>::step(A[rb], B[cb], acc[rb][cb]);
  }
}

// Sum the per-wave accumulators of KS waves that split the reduction, in a
// fixed wave order (bit-reproducible).  Wave 0 ends up with the total.
template <int KS, int NFRAG>
SIMSD_DEV void reduce_waves(f32x4_t (&acc)[NFRAG], int wave_k, int lane, float* red /* LDS */) {
  if (KS == 1) return;
  // red layout: [KS-1][NFRAG*4][64]
  if (wave_k > 0) {
#pragma unroll
    for (int f = 0; f < NFRAG; ++f)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[((wave_k - 1) * NFRAG * 4 + f * 4 + j) * 64 + lane] = acc[f][j];
  }
  __syncthreads();
  if (wave_k == 0) {
    for (int w = 1; w < KS; ++w)
#pragma unroll
      for (int f = 0; f < NFRAG; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[f][j] += red[((w - 1) * NFRAG * 4 + f * 4 + j) * 64 + lane];
  }
}

}  // namespace simsd

// ---------------------------------------------------------------- host errors
namespace simsd {
int set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace simsd

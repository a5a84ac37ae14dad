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

// fp16 roundings take their operand as a value already rounded to fp32, as
// torch computes an fp16 op (in fp32, then .to(fp16)).  Without the empty
// register constraint the compiler may fuse a preceding fp32 multiply or add
// into the conversion (v_fma_mixlo_f16: one rounding, straight to fp16),
// which differs from the two roundings in rare cases -- and differently from
// one kernel to the next, depending on where it applies it.
SIMSD_DEV float keep_f32(float v) {
  asm("" : "+v"(v));
  return v;
}

template <int DT> SIMSD_DEV void store_elem(char* base, int64_t idx, float v);
template <> SIMSD_DEV void store_elem<kBF16>(char* base, int64_t idx, float v) {
  reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16_bits(v);
}
template <> SIMSD_DEV void store_elem<kF16>(char* base, int64_t idx, float v) {
  reinterpret_cast<_Float16*>(base)[idx] = (_Float16)keep_f32(v);
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
template <> SIMSD_DEV float round_to<kF16>(float v) { return (float)(_Float16)keep_f32(v); }
template <> SIMSD_DEV float round_to<kF32>(float v) { return v; }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// 16-bit storage element <-> float (the low half of a packed pair first).
template <int DT> SIMSD_DEV float h16_to_f32(uint32_t h);
template <> SIMSD_DEV float h16_to_f32<kBF16>(uint32_t h) { return bf16_bits_to_f32(h & 0xffffu); }
template <> SIMSD_DEV float h16_to_f32<kF16>(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}
template <int DT> SIMSD_DEV uint32_t f32_to_h16(float v);
template <> SIMSD_DEV uint32_t f32_to_h16<kBF16>(float v) { return f32_to_bf16_bits(v); }
template <> SIMSD_DEV uint32_t f32_to_h16<kF16>(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)keep_f32(v));
}

// RMSNorm of 8 packed 16-bit values: out = dtype(gamma * dtype(x * r)), the
// rounding points of the stock PyTorch RMSNorm (x * rsqrt(mean(x^2) + eps)
// in fp32, cast to the input dtype, times the weight in that dtype).
template <int DT>
SIMSD_DEV u32x4_t rms_scale8(u32x4_t x, u32x4_t g, float r) {
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w}, gv[4] = {g.x, g.y, g.z, g.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = round_to<DT>(h16_to_f32<DT>(gv[i]) * round_to<DT>(h16_to_f32<DT>(xv[i]) * r));
    const float hi = round_to<DT>(h16_to_f32<DT>(gv[i] >> 16) * round_to<DT>(h16_to_f32<DT>(xv[i] >> 16) * r));
    o[i] = f32_to_h16<DT>(lo) | (f32_to_h16<DT>(hi) << 16);
  }
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

// bf16: both roundings of a pair in one v_cvt_pk_bf16_f32 each (round to
// nearest even, as the software rounding above).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <>
SIMSD_DEV u32x4_t rms_scale8<kBF16>(u32x4_t x, u32x4_t g, float r) {
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w}, gv[4] = {g.x, g.y, g.z, g.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2_t xf = {__uint_as_float(xv[i] << 16), __uint_as_float(xv[i] & 0xffff0000u)};
    const uint32_t t = __builtin_bit_cast(uint32_t, __builtin_convertvector(xf * r, bf16x2_t));
    const f32x2_t tf = {__uint_as_float(t << 16), __uint_as_float(t & 0xffff0000u)};
    const f32x2_t gf = {__uint_as_float(gv[i] << 16), __uint_as_float(gv[i] & 0xffff0000u)};
    o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(gf * tf, bf16x2_t));
  }
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

// Sum of squares of 8 packed 16-bit values, in element order.
template <int DT>
SIMSD_DEV float sumsq8(u32x4_t x, float acc) {
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = h16_to_f32<DT>(xv[i]), hi = h16_to_f32<DT>(xv[i] >> 16);
    acc += lo * lo;
    acc += hi * hi;
  }
  return acc;
}

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

// ------------------------------------------------- MFMA 4x4x4, 16 blocks
// v_mfma_f32_4x4x4_16b_{bf16,f16}: 16 independent 4x4x4 products.
//   A: lane l holds block b = l/4, row i = l%4, its 4 k values
//   B: lane l holds block b = l/4, col j = l%4, its 4 k values
//   D: lane l holds block b = l/4, col j = l%4, rows i = 0..3 in 4 registers
// Used for M <= 8 GEMV: A rows are 4 weight rows, B cols are up to 4 tokens,
// and the 16 blocks are 16 consecutive 4-element k chunks, so one 16-byte
// load per lane covers 4 rows x 256 contiguous bytes (two MFMAs' worth).
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <int DT> struct Mfma4;
template <> struct Mfma4<kBF16> {
  static SIMSD_DEV f32x4_t step(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                  __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  }
};
template <> struct Mfma4<kF16> {
  static SIMSD_DEV f32x4_t step(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4_t, a),
                                              __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  }
};

SIMSD_DEV u32x2_t lo2(u32x4_t v) { return u32x2_t{v.x, v.y}; }
SIMSD_DEV u32x2_t hi2(u32x4_t v) { return u32x2_t{v.z, v.w}; }

SIMSD_DEV u32x4_t zero4() { return u32x4_t{0u, 0u, 0u, 0u}; }

// ------------------------------------------ fast accumulate (buffer loads)
// Operands are read through buffer resources (one uniform descriptor per A
// block and one for B) with per-lane 32-bit byte offsets.  An offset at or past
// the descriptor's extent reads as zero in hardware, which covers the K tail,
// weight rows past N, activation rows past M and empty slots -- so the loads
// are unconditional, carry no branches, and the compiler can keep the next
// batch in flight while the current one feeds the MFMAs.
// Requirements: 16-byte aligned bases, row strides and row length Kb (bytes)
// multiples of 16, every extent below kOob.
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef i32x4_t rsrc_t;                       // V# buffer descriptor, 4 dwords
constexpr uint32_t kOob = 0xFFFFFFF0u;        // never inside a valid extent
constexpr int kRsrcWord3 = 0x00020000;        // raw 32-bit buffer, gfx9 family
constexpr int kAuxStream = 2;                 // nt: streamed once, do not keep
constexpr int kAuxKeep = 0;

// The LLVM intrinsic, bound by name: (descriptor, voffset, soffset, cache bits).
__device__ i32x4_t simsd_raw_buffer_load_v4i32(i32x4_t rsrc, int32_t voffset, int32_t soffset,
                                               int32_t aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");

SIMSD_DEV rsrc_t make_rsrc(const void* base, uint32_t extent_bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  // word1 high half = stride 0; word3 = raw dword format
  return rsrc_t{(int32_t)(uint32_t)p, (int32_t)(uint32_t)((p >> 32) & 0xFFFFu),
                (int32_t)extent_bytes, kRsrcWord3};
}

template <int AUX>
SIMSD_DEV u32x4_t buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, simsd_raw_buffer_load_v4i32(r, (int32_t)off, 0, AUX));
}

// The same for 4 bytes.
__device__ int32_t simsd_raw_buffer_load_i32(i32x4_t rsrc, int32_t voffset, int32_t soffset, int32_t aux)
    __asm("llvm.amdgcn.raw.buffer.load.i32");

template <int AUX = 0>
SIMSD_DEV uint32_t buf_load4(rsrc_t r, uint32_t off) {
  return (uint32_t)simsd_raw_buffer_load_i32(r, (int32_t)off, 0, AUX);
}

// sc0 | sc1: a load that misses every cache level (reads what another XCD
// wrote through to memory)
constexpr int kAuxThrough = 17;

template <int RB, int CB, int U>
SIMSD_DEV void load_batch(u32x4_t (&A)[U][RB], u32x4_t (&B)[U][CB], const rsrc_t (&ra)[RB],
                          const uint32_t (&aoff)[RB], rsrc_t rb_, const uint32_t (&boff)[CB],
                          const bool (&bok)[CB], int s, int s1, uint32_t lane_off, uint32_t Kb) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t k = (uint32_t)(s + u) * kStepBytes + lane_off;
    const bool ok = (s + u < s1) && (k < Kb);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      A[u][rb] = buf_load16<kAuxStream>(ra[rb], ok ? aoff[rb] + k : kOob);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
      B[u][cb] = buf_load16<kAuxKeep>(rb_, (ok && bok[cb]) ? boff[cb] + k : kOob);
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

// Sums k-steps [s0, s1) (64 bytes of every row each) into acc, U steps per
// batch: the batch's loads all issue back to back, and each MFMA waits only
// for its own operands (graduated vmcnt), so the batch streams through.
template <int DT, int RB, int CB, int U>
SIMSD_DEV void accum_fast(const rsrc_t (&ra)[RB], const uint32_t (&aoff)[RB], rsrc_t rb_,
                          const uint32_t (&boff)[CB], const bool (&bok)[CB], int s0, int s1,
                          uint32_t lane_off, uint32_t Kb, f32x4_t (&acc)[RB][CB]) {
  for (int s = s0; s < s1; s += U) {
    u32x4_t A[U][RB], B[U][CB];
    load_batch<RB, CB, U>(A, B, ra, aoff, rb_, boff, bok, s, s1, lane_off, Kb);
    // keep every load of the batch ahead of its first MFMA (the scheduler
    // would otherwise interleave them to save registers and cut the loads
    // in flight)
    __builtin_amdgcn_sched_barrier(0);
    mfma_batch<DT, RB, CB, U>(A, B, acc);
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

// ------------------------------------------- LDS-relayout MFMA accumulation
// acc[rb][cb] += A_rb . B_cb^T over the 256-byte k chunks [c0, c1) with
// v_mfma_f32_16x16x32.  Weight block rb (16 rows, descriptor ra[rb], row 0 at
// byte a_row0[rb], row stride a_sn[rb]) is read as 4 rows x 256 contiguous
// bytes per load instruction (lane l: row 4q + l/16, bytes 16*(l%16)), written
// to the wave's own LDS tile (16*RB rows, row stride kLdsRow = 272 B: no bank
// conflicts for the 16-byte writes or for the MFMA-layout reads) and read back
// in the A layout.  B block cb is loaded in the B layout straight from memory:
// lane (g, r) reads 16 bytes at boff[cb] + k + 16 g of its row r (invalid rows
// and bytes past Kb read zero).  U chunks are loaded per batch, all before the
// first LDS write.  A wave's LDS accesses complete in order, so the reads see
// the writes and the next chunk's writes follow the reads: no barrier.  Rows at
// or past VR (a tile of fewer than 16 RB rows) are not loaded: their LDS rows
// are written with zeros and their outputs are never stored.
constexpr int kStep4Bytes = 256;            // bytes of one row per 4-row load step
constexpr int kLdsRow = kStep4Bytes + 16;   // padded LDS row of a 256 B chunk
// LDS per workgroup on gfx950 (CDNA4); the library is built for gfx950 only,
// and some tiles use more than the 64 KiB of earlier CDNA parts.
constexpr int kLdsBytesGfx950 = 160 * 1024;

template <int DT, int RB, int CB, int U, int VR = 16 * RB>
SIMSD_DEV void accum_lds(const rsrc_t (&ra)[RB], const uint32_t (&a_row0)[RB],
                         const uint32_t (&a_sn)[RB], rsrc_t rbx, const uint32_t (&boff)[CB],
                         const bool (&bok)[CB], int c0, int c1, uint32_t Kb, char* tile,
                         f32x4_t (&acc)[RB][CB]) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, r = lane & 15;     // MFMA operand layout
  const int lr = lane >> 4, lc = lane & 15;   // loader layout: row l/16 of 4, chunk l%16
  for (int c = c0; c < c1; c += U) {
    u32x4_t W[U][RB][4], B[U][4][CB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = c + u < c1;
      const uint32_t kc = (uint32_t)(c + u) * kStep4Bytes;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t k = kc + lc * kLaneBytes;
          if (16 * rb + 4 * q < VR)
            W[u][rb][q] = buf_load16<kAuxStream>(
                ra[rb], live && k < Kb ? a_row0[rb] + (uint32_t)(4 * q + lr) * a_sn[rb] + k : kOob);
          else
            W[u][rb][q] = zero4();
        }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const uint32_t k = kc + j * kStepBytes + g * kLaneBytes;
          B[u][j][cb] = buf_load16<kAuxKeep>(rbx, live && bok[cb] && k < Kb ? boff[cb] + k : kOob);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<u32x4_t*>(tile + (16 * rb + 4 * q + lr) * kLdsRow + lc * kLaneBytes) = W[u][rb][q];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x4_t A[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          A[rb] = *reinterpret_cast<const u32x4_t*>(tile + (16 * rb + r) * kLdsRow + j * kStepBytes +
                                                    g * kLaneBytes);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = Mfma<DT>::step(A[rb], B[u][j][cb], acc[rb][cb]);
      }
    }
  }
}

// accum_lds with the B operand staged the same way: B block cb is 16
// consecutive rows of one matrix (rows 16 cb .. 16 cb + 15, stride b_sn bytes,
// rows >= b_rows read zero), loaded as 4 rows x 256 B per instruction into
// LDS rows 16 RB + 16 cb + ... of the wave's tile and read back in the B
// layout.  Whole cache lines per load instead of 64 bytes of 16 rows, for
// activations that every workgroup re-reads from L2.  The tile holds
// 16 (RB + CB) rows.  Weight rows at or past VR are not loaded, as in
// accum_lds.
template <int DT, int RB, int CB, int U, int VR = 16 * RB>
SIMSD_DEV void accum_lds_ab(const rsrc_t (&ra)[RB], const uint32_t (&a_row0)[RB],
                            const uint32_t (&a_sn)[RB], rsrc_t rbx, uint32_t b_sn, int b_rows, int c0,
                            int c1, uint32_t Kb, char* tile, f32x4_t (&acc)[RB][CB]) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, r = lane & 15;     // MFMA operand layout
  const int lr = lane >> 4, lc = lane & 15;   // loader layout: row l/16 of 4, chunk l%16
  for (int c = c0; c < c1; c += U) {
    u32x4_t W[U][RB][4], X[U][CB][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = c + u < c1;
      const uint32_t k = (uint32_t)(c + u) * kStep4Bytes + lc * kLaneBytes;
      const bool kok = live && k < Kb;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          W[u][rb][q] = 16 * rb + 4 * q < VR
                            ? buf_load16<kAuxStream>(
                                  ra[rb], kok ? a_row0[rb] + (uint32_t)(4 * q + lr) * a_sn[rb] + k : kOob)
                            : zero4();
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = 16 * cb + 4 * q + lr;
          X[u][cb][q] = buf_load16<kAuxKeep>(rbx, kok && row < b_rows ? (uint32_t)row * b_sn + k : kOob);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<u32x4_t*>(tile + (16 * rb + 4 * q + lr) * kLdsRow + lc * kLaneBytes) = W[u][rb][q];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<u32x4_t*>(tile + (16 * (RB + cb) + 4 * q + lr) * kLdsRow + lc * kLaneBytes) =
              X[u][cb][q];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x4_t A[RB], B[CB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          A[rb] = *reinterpret_cast<const u32x4_t*>(tile + (16 * rb + r) * kLdsRow + j * kStepBytes +
                                                    g * kLaneBytes);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          B[cb] = *reinterpret_cast<const u32x4_t*>(tile + (16 * (RB + cb) + r) * kLdsRow +
                                                    j * kStepBytes + g * kLaneBytes);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = Mfma<DT>::step(A[rb], B[cb], acc[rb][cb]);
      }
    }
  }
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for every global load the wave has in flight, which drains a
// prefetch issued ahead of the barrier; these fences are scoped to LDS.
SIMSD_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
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

// ------------------------------------------------------- wave all-reduces
// Lane exchanges without LDS: DPP quad permutes (lane xor 1, xor 2), DPP row
// rotations by 4 and 8 (which, after the quad stages, cover a 16-lane row),
// and the gfx950 swaps v_permlane16_swap / v_permlane32_swap, which applied
// to (v, v) return the values of both rows of a row pair (both half-waves):
// combining the two outputs in a fixed order gives every lane the same result.
SIMSD_DEV int dpp_quad_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
SIMSD_DEV int dpp_quad_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }
SIMSD_DEV int dpp_row_ror4(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false); }
SIMSD_DEV int dpp_row_ror8(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false); }

// Combine(a, b) must be commutative for the in-row stages; the result of the
// last two stages is combine(lower half, upper half) on every lane.
template <typename Combine>
SIMSD_DEV float wave_allreduce(float v, Combine combine) {
  v = combine(v, __int_as_float(dpp_quad_xor1(__float_as_int(v))));
  v = combine(v, __int_as_float(dpp_quad_xor2(__float_as_int(v))));
  v = combine(v, __int_as_float(dpp_row_ror4(__float_as_int(v))));
  v = combine(v, __int_as_float(dpp_row_ror8(__float_as_int(v))));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = combine(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = combine(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  // the in-row stages may associate differently per lane: take lane 0's value
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// Sum NV per-lane values over lane bits 5, 4 and the row bits from log2(LO)
// up to 3.  Bits 5 and 4 by reduce-scatter on the gfx950 lane swaps:
// v_permlane32_swap(a, b) leaves [a.lo, b.lo] / [a.hi, b.hi], so one swap and
// one add sum a pair of values over the two half-waves and keep one of them
// per half (likewise rows 0/1 and 2/3 with v_permlane16_swap).  The row bits
// by adding row rotations by 8, 4, ..., LO (after which every lane of the
// rotation class holds the full sum).  Afterwards lane l holds, in val[p] for
// p < NV/4, the sum of original value p + bit5(l) * NV/2 + bit4(l) * NV/4.
// A fixed instruction sequence: bit-reproducible.
template <int NV, int LO>
__device__ __forceinline__ void reduce_lanes(float (&val)[NV]) {
  static_assert(NV >= 4 && (NV & (NV - 1)) == 0, "power of two >= 4");
  static_assert(LO == 1 || LO == 2 || LO == 4 || LO == 8, "rotation");
#pragma unroll
  for (int p = 0; p < NV / 2; ++p) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(val[p]),
                                                    __float_as_uint(val[p + NV / 2]), false, false);
    val[p] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int p = 0; p < NV / 4; ++p) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(val[p]),
                                                    __float_as_uint(val[p + NV / 4]), false, false);
    val[p] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int p = 0; p < NV / 4; ++p) {
    val[p] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(val[p]), 0x128, 0xF, 0xF, false));
    if (LO <= 4)
      val[p] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(val[p]), 0x124, 0xF, 0xF, false));
    if (LO <= 2)
      val[p] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(val[p]), 0x122, 0xF, 0xF, false));
    if (LO <= 1)
      val[p] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(val[p]), 0x121, 0xF, 0xF, false));
  }
}

SIMSD_DEV float wave_max(float v) {
  return wave_allreduce(v, [](float a, float b) { return fmaxf(a, b); });
}
SIMSD_DEV float wave_sum(float v) {
  return wave_allreduce(v, [](float a, float b) { return a + b; });
}

// Inclusive prefix sum over the wave's 64 lanes, in DPP moves (no LDS
// permutes): shifts by 1, 2, 4 and 8 within each 16-lane row, then the
// totals of rows 0 and 2 added to rows 1 and 3 (row_bcast:15) and the running
// total of rows 0-1 to rows 2 and 3 (row_bcast:31).  Lanes outside a move's
// source or row mask add 0.
SIMSD_DEV int wave_inclusive_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);   // row_bcast:15, rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);   // row_bcast:31, rows 2 and 3
  return v;
}

// Largest 64-bit key over the wave, on every lane.  Route keys are
// (order-preserving bits of the logit) << 32 | ~index, so the maximum is the
// largest logit and, among equal logits, the lowest index; 0 marks an entry
// that is taken or absent.
SIMSD_DEV uint32_t float_order_bits(float f) {
  uint32_t b = __float_as_uint(f);
  if (b == 0x80000000u) b = 0u;   // -0 == +0: equal keys, so ties go by index
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
SIMSD_DEV float float_from_order_bits(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
SIMSD_DEV uint64_t wave_max_u64(uint64_t key) {
  auto take = [&](uint32_t lo, uint32_t hi) {
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    key = o > key ? o : key;
  };
  auto lo = [&]() { return (int)(uint32_t)key; };
  auto hi = [&]() { return (int)(uint32_t)(key >> 32); };
  take((uint32_t)dpp_quad_xor1(lo()), (uint32_t)dpp_quad_xor1(hi()));
  take((uint32_t)dpp_quad_xor2(lo()), (uint32_t)dpp_quad_xor2(hi()));
  take((uint32_t)dpp_row_ror4(lo()), (uint32_t)dpp_row_ror4(hi()));
  take((uint32_t)dpp_row_ror8(lo()), (uint32_t)dpp_row_ror8(hi()));
  {
    const auto l = __builtin_amdgcn_permlane16_swap((uint32_t)lo(), (uint32_t)lo(), false, false);
    const auto h = __builtin_amdgcn_permlane16_swap((uint32_t)hi(), (uint32_t)hi(), false, false);
    key = ((uint64_t)h[0] << 32) | l[0];
    take(l[1], h[1]);
  }
  {
    const auto l = __builtin_amdgcn_permlane32_swap((uint32_t)lo(), (uint32_t)lo(), false, false);
    const auto h = __builtin_amdgcn_permlane32_swap((uint32_t)hi(), (uint32_t)hi(), false, false);
    key = ((uint64_t)h[0] << 32) | l[0];
    take(l[1], h[1]);
  }
  return key;
}

}  // namespace simsd

// ---------------------------------------------------------------- host errors
namespace simsd {
int set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace simsd

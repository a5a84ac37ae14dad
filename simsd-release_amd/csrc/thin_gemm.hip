// Skinny GEMM y[M,N] = x[M,K] . w[N,K]^T (+ bias) for gfx950.
//
// Replaces the Triton _thin_gemv_kernel / _thin_gemv_reduce pair of
// kernels/thin_linear_fused.py:67-171 (reference).  The op streams the weight
// once from HBM; three kernels cover the token counts:
//   * thin_gemv4_kernel (M <= 8, bf16/fp16): v_mfma_f32_4x4x4_16b with the
//     tokens as the 4 output columns, weight read as 4 rows x 256 contiguous
//     bytes per instruction, activations held in registers;
//   * thin_gemm_lds_kernel (M > 8, bf16/fp16): v_mfma_f32_16x16x32 with the
//     same weight access, the tile re-laid out through LDS into the MFMA A
//     operand;
//   * thin_gemm_kernel (fp32, strided or unaligned views): 16x16 MFMA with
//     the operands loaded directly in MFMA layout (below 16 rows per
//     workgroup the A rows repeat and the duplicates' outputs are dropped).
// A workgroup owns 4..32 weight rows and splits K across its waves, whose fp32
// partials meet in LDS in fixed wave order.  An explicit split along K
// (SPLIT > 1) writes fp32 partial tiles and a second launch sums them in split
// order: deterministic, no atomics, no cross-workgroup synchronisation.
#include <mutex>
#include <type_traits>

#include "simsd_common.hpp"
#include "simsd_kernels.h"

#ifndef SIMSD_THIN_U
#define SIMSD_THIN_U 8   // k-steps per batch at one A and one B block
#endif
#ifndef SIMSD_LDS_X
#define SIMSD_LDS_X 1    // 9..32 tokens: stage the activations through LDS too
#endif


namespace simsd {

struct ThinArgs {
  const char* x;
  int64_t sxm, sxk;          // element strides
  const char* w;
  int64_t swn, swk;
  const char* bias;          // nullable, element stride sb
  int64_t sb;
  char* y;
  int64_t sym, syn;
  float* part;               // [split][M][N] fp32 partials when split > 1 ([split][M][2N] gated)
  const char* w2;            // gated (SiLU-mul) kernels: the up matrix, row stride sw2n
  int64_t sw2n;
  const char* gamma;         // RMSNorm prologue: weight [K] (contiguous), epsilon
  float eps;
  const char* res;           // residual added to the rounded output (nullable), strides srm, srn
  int64_t srm, srn;
  int64_t M, N, K;           // gated: N = output columns (rows of each of w, w2)
  int steps;                 // ceil(K * esize / 64)
  int steps_per_split;
};

template <int DT, int RT, int RB, int CB, int KS, int U, bool FAST, bool PARTIAL>
__global__ __launch_bounds__(64 * KS) void thin_gemm_kernel(ThinArgs a) {
  static_assert(RT == 4 || RT == 8 || RT == 16, "rows per block");
  static_assert(RT == 16 || RB == 1, "sub-16-row tiles use one block");
  constexpr int ES = DTypeInfo<DT>::kSize;
  constexpr int NF = RB * CB;
  const int lane = threadIdx.x & 63;
  const int wk = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t n_tile = (int64_t)blockIdx.x * (RT * RB);
  const int64_t m_tile = (int64_t)blockIdx.z * (CB * 16);
  const int split_id = blockIdx.y;

  // k-steps of this workgroup, then of this wave
  const int s_lo = split_id * a.steps_per_split;
  const int s_hi = min(a.steps, s_lo + a.steps_per_split);
  const int span = max(0, s_hi - s_lo);
  const int per_w = (span + KS - 1) / KS;
  const int w0 = s_lo + wk * per_w;
  const int w1 = min(s_hi, w0 + per_w);

  f32x4_t acc[RB][CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (FAST) {
    // One descriptor over this tile's weight rows and one over its activation
    // rows; rows past N or M fall outside the extents and read as zero.
    const uint32_t Kb = (uint32_t)(a.K * ES);
    const uint32_t swn_b = (uint32_t)(a.swn * ES), sxm_b = (uint32_t)(a.sxm * ES);
    const int64_t rows_valid = min((int64_t)(RT * RB), a.N - n_tile);
    const int64_t cols_valid = min((int64_t)(CB * 16), a.M - m_tile);
    const rsrc_t rA = make_rsrc(a.w + n_tile * a.swn * ES, (uint32_t)(rows_valid - 1) * swn_b + Kb);
    const rsrc_t rB = make_rsrc(a.x + m_tile * a.sxm * ES, (uint32_t)(cols_valid - 1) * sxm_b + Kb);
    rsrc_t ra[RB];
    uint32_t aoff[RB], boff[CB];
    bool bok[CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      ra[rb] = rA;
      aoff[rb] = (uint32_t)(rb * RT + (r % RT)) * swn_b;
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      boff[cb] = (uint32_t)(cb * 16 + r) * sxm_b;
      bok[cb] = cb * 16 + r < cols_valid;
    }
    accum_fast<DT, RB, CB, U>(ra, aoff, rB, boff, bok, w0, w1, (uint32_t)(g * kLaneBytes), Kb, acc);
  } else {
    const char* arow[RB];
    const char* brow[CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int64_t n = min(n_tile + rb * RT + (r % RT), a.N - 1);
      arow[rb] = a.w + n * a.swn * ES;
    }
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int64_t m = m_tile + cb * 16 + r;
      brow[cb] = m < a.M ? a.x + m * a.sxm * ES : nullptr;
    }
    accum_generic<DT, RB, CB>(arow, a.swk * ES, brow, a.sxk * ES, w0, w1, g, a.K, acc);
  }

  __shared__ float red[KS > 1 ? (KS - 1) * NF * 4 * 64 : 1];
  reduce_waves<KS, NF>(reinterpret_cast<f32x4_t(&)[NF]>(acc), wk, lane, red);
  if (wk != 0 || 4 * g >= RT) return;   // lanes of duplicated rows hold no new output

#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int64_t m = m_tile + cb * 16 + r;
      const int64_t nb = n_tile + rb * RT + 4 * g;
      if (m < a.M) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t n = nb + j;
          if (n < a.N) {
            float v = acc[rb][cb][j];
            if (PARTIAL) {
              a.part[((int64_t)split_id * a.M + m) * a.N + n] = v;
            } else {
              if (a.bias != nullptr) v = round_to<DT>(v) + load_elem<DT>(a.bias, n * a.sb);
              if (a.res != nullptr) v = round_to<DT>(v) + load_elem<DT>(a.res, m * a.srm + n * a.srn);
              store_elem<DT>(a.y, m * a.sym + n * a.syn, v);
            }
          }
        }
      }
    }
}

// ---------------------------------------------------------------------------
// M <= 8 GEMV on v_mfma_f32_4x4x4_16b: the weight is read as 4 rows x 256
// contiguous bytes per wave instruction (two full cache lines per row), the
// activation chunk for the wave's K range sits in registers and is reused by
// every 4-row group, so the inner loop issues weight loads only.
//   RW  weight rows per workgroup (4..32), G = RW / 4 row groups
//   MS  column sets of 4 tokens (1: M <= 4, 2: M <= 8)
//   KS  waves per workgroup splitting K
//   CH  load steps (128 k elements each) whose activations are held at once
//   GB  row groups whose loads are issued together

// Gated output: h = dtype(dtype(silu(dtype(g))) * dtype(u)), the rounding
// points of a bf16 act_fn(gate_proj(x)) * up_proj(x) in PyTorch.
template <int DT>
SIMSD_DEV float silu_mul(float g, float u) {
  const float gr = round_to<DT>(g);
  const float sv = round_to<DT>(gr / (1.f + expf(-gr)));
  return sv * round_to<DT>(u);
}

// Write one output (or its split partial).  Gated: g at column n, u at
// column N + n of the partial row.
template <int DT, bool PARTIAL, bool GLU>
SIMSD_DEV void put_out(const ThinArgs& a, int split_id, int64_t m, int64_t n, float v, float u) {
  if (PARTIAL) {
    const int64_t row = ((int64_t)split_id * a.M + m) * (GLU ? 2 * a.N : a.N);
    a.part[row + n] = v;
    if (GLU) a.part[row + a.N + n] = u;
  } else if (GLU) {
    store_elem<DT>(a.y, m * a.sym + n * a.syn, silu_mul<DT>(v, u));
  } else {
    // bias: the product rounded to the dtype, then the dtype add -- the
    // reference's y += bias on the kernel's output
    if (a.bias != nullptr) v = round_to<DT>(v) + load_elem<DT>(a.bias, n * a.sb);
    // residual: the projection rounded to the dtype, then the dtype add
    if (a.res != nullptr) v = round_to<DT>(v) + load_elem<DT>(a.res, m * a.srm + n * a.srn);
    store_elem<DT>(a.y, m * a.sym + n * a.syn, v);
  }
}

// column sets of 4 tokens up to which the norm runs inside the GEMV (2: the
// GEMV's whole range; at 8 tokens fused is 1.4-1.5 us faster than norm + GEMV)
#ifndef SIMSD_NORM_MAX_MS
#define SIMSD_NORM_MAX_MS 2
#endif
constexpr int kNormMaxMs = SIMSD_NORM_MAX_MS;
// Every workgroup of the fused form reads its tokens' whole rows for the
// statistics.  Past this many bytes of such reads in one call (an lm_head's
// ~9.5K workgroups read 152 MB at 4 tokens) a separate norm launch is cheaper.
#ifndef SIMSD_NORM_STATS_BUDGET
#define SIMSD_NORM_STATS_BUDGET (32ll << 20)
#endif


// statistics passes of the norm prologue issued ahead of the first weights
#ifndef SIMSD_NORM_EARLY
#define SIMSD_NORM_EARLY 2
#endif

// The fields the first loads depend on come as separate scalar arguments
// ahead of ThinArgs: the build preloads leading scalar kernel arguments into
// SGPRs (-amdgpu-kernarg-preload-count), so the first weight and activation
// loads wait for no kernarg fetch.  Kb, swn_b, sxm_b, sw2n_b: K and the row
// strides in bytes; the rest of ThinArgs is read where it is used.
template <int DT, int RW, int MS, int KS, int CH, int GB, bool PARTIAL, bool GLU, bool NORM>
__global__ __launch_bounds__(64 * KS) void thin_gemv4_kernel(const char* __restrict__ w, const char* __restrict__ x,
                                                             const char* __restrict__ w2, uint32_t Kb, uint32_t swn_b,
                                                             uint32_t sxm_b, uint32_t sw2n_b, int N, int M, int steps,
                                                             int steps_per_split, ThinArgs a) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  constexpr int G = RW / 4;
  static_assert(RW % 4 == 0 && G % GB == 0, "row groups");
  static_assert(!GLU || (G % 2 == 0 && (G / 2) % GB == 0), "gated: gate and up halves of whole batches");
  // gated: groups [0, G/2) are gate rows, [G/2, G) the same rows of up
  constexpr int OUT = GLU ? RW / 2 : RW;   // output columns per workgroup
  const int lane = threadIdx.x & 63;
  const int wk = threadIdx.x >> 6;
  const int i4 = lane & 3;          // A row / B column within a block
  const int b4 = lane >> 2;         // 4x4x4 block = 8-element k chunk of a load step
  const int64_t n_tile = (int64_t)blockIdx.x * OUT;
  const int64_t m_tile = (int64_t)blockIdx.z * (4 * MS);
  const int split_id = blockIdx.y;

  const int s_lo = split_id * steps_per_split;
  const int s_hi = min(steps, s_lo + steps_per_split);
  const int span = max(0, s_hi - s_lo);
  const int per_w = (span + KS - 1) / KS;
  const int w0 = s_lo + wk * per_w;
  const int w1 = min(s_hi, w0 + per_w);

  const int64_t rows_valid = min((int64_t)OUT, (int64_t)N - n_tile);
  const int64_t cols_valid = min((int64_t)(4 * MS), (int64_t)M - m_tile);
  const rsrc_t rA = make_rsrc(w + n_tile * swn_b, (uint32_t)(rows_valid - 1) * swn_b + Kb);
  const rsrc_t rA2 = GLU ? make_rsrc(w2 + n_tile * sw2n_b, (uint32_t)(rows_valid - 1) * sw2n_b + Kb) : rA;
  const rsrc_t rB = make_rsrc(x + m_tile * sxm_b, (uint32_t)(cols_valid - 1) * sxm_b + Kb);
  const uint32_t lane_k = (uint32_t)(b4 * kLaneBytes);

  // RMSNorm prologue: every workgroup derives the scale of its <= 8 tokens
  // from their whole rows (L2-resident after the first workgroup), then
  // normalises the activations as they are loaded.  rr[c]: this lane's token
  // 4c + i4.
  float rr[MS];
  rsrc_t rG{};
  // weight rows of this wave's first chunk: A operands for group g, step s
  auto load_a = [&](int c0, int g, int s) {
    const int c_lim = min(w1, c0 + CH);
    const bool up = GLU && g >= G / 2;
    const uint32_t roff = (uint32_t)(4 * (up ? g - G / 2 : g) + i4) * (up ? sw2n_b : swn_b);
    const uint32_t k = (uint32_t)(c0 + s) * kStep4Bytes + lane_k;
    const bool ok = (c0 + s < c_lim) && (k < Kb);
    return buf_load16<kAuxStream>(up ? rA2 : rA, ok ? roff + k : kOob);
  };
  // activations (token 4c + i4) and gamma of step s of the chunk at c0
  auto load_b = [&](int c0, int s, int c) {
    const int c_lim = min(w1, c0 + CH);
    const uint32_t k = (uint32_t)(c0 + s) * kStep4Bytes + lane_k;
    const bool ok = (c0 + s < c_lim) && (k < Kb) && (4 * c + i4 < cols_valid);
    return buf_load16<kAuxKeep>(rB, ok ? (uint32_t)(4 * c + i4) * sxm_b + k : kOob);
  };
  auto load_g = [&](int c0, int s) {
    const int c_lim = min(w1, c0 + CH);
    const uint32_t k = (uint32_t)(c0 + s) * kStep4Bytes + lane_k;
    return buf_load16<kAuxKeep>(rG, (c0 + s < c_lim) && (k < Kb) ? k : kOob);
  };
  // small chunks: the first chunk's activations and gamma are requested with
  // the statistics, so that they are in registers when the scale is known
  constexpr bool kPreB = NORM && CH <= 2;
  u32x4_t B0[kPreB ? CH : 1][MS], G0[kPreB ? CH : 1];
  // With the norm prologue the statistics loads of the first kNormEarly
  // passes go out first, then the first chunk's weights, so that the wait for
  // the statistics (loads complete in issue order) does not also wait for the
  // weights, whose latency then overlaps the norm.
  u32x4_t A0[NORM ? G : 1][NORM ? CH : 1];
  if constexpr (NORM) {
    rG = make_rsrc(a.gamma, Kb);
    constexpr int MT = 4 * MS;
    constexpr int kNormEarly = SIMSD_NORM_EARLY;
    const uint32_t x_stride = 64 * KS * kLaneBytes;
    const uint32_t x_off = (uint32_t)threadIdx.x * kLaneBytes;
    __shared__ float ssq_red[KS][MT];
    float ssq[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) ssq[j] = 0.f;
    u32x4_t v0[kNormEarly][MT];
#pragma unroll
    for (int i = 0; i < kNormEarly; ++i) {
      const uint32_t off = x_off + i * x_stride;
#pragma unroll
      for (int j = 0; j < MT; ++j)
        v0[i][j] = buf_load16<kAuxKeep>(rB, (j < cols_valid && off < Kb) ? (uint32_t)j * sxm_b + off : kOob);
    }
    if constexpr (kPreB) {
#pragma unroll
      for (int st = 0; st < CH; ++st) {
#pragma unroll
        for (int c = 0; c < MS; ++c) B0[st][c] = load_b(w0, st, c);
        G0[st] = load_g(w0, st);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int st = 0; st < CH; ++st) A0[g][st] = load_a(w0, g, st);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kNormEarly; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) ssq[j] = sumsq8<DT>(v0[i][j], ssq[j]);
    for (uint32_t off = x_off + kNormEarly * x_stride; off < Kb; off += x_stride) {
      u32x4_t v[MT];
#pragma unroll
      for (int j = 0; j < MT; ++j) v[j] = buf_load16<kAuxKeep>(rB, j < cols_valid ? (uint32_t)j * sxm_b + off : kOob);
#pragma unroll
      for (int j = 0; j < MT; ++j) ssq[j] = sumsq8<DT>(v[j], ssq[j]);
    }
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const float t = wave_sum(ssq[j]);
      if (lane == 0) ssq_red[wk][j] = t;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < MS; ++c) {
      float t = 0.f;
      for (int w = 0; w < KS; ++w) t += ssq_red[w][4 * c + i4];
      rr[c] = 1.f / sqrtf(t / (float)a.K + a.eps);
    }
  }

  f32x4_t acc[G][MS];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int c = 0; c < MS; ++c) acc[g][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // one chunk: get_b / get_g / get_a give the activations, gamma and weight
  // operands of step s (token set c, row group g)
  auto run_chunk = [&](int c0, auto&& get_b, auto&& get_g, auto&& get_a) {
    // activations of this chunk: lane (j, b) holds token 4c+j, k chunk b
    u32x4_t B[CH][MS];
#pragma unroll
    for (int s = 0; s < CH; ++s) {
#pragma unroll
      for (int c = 0; c < MS; ++c) B[s][c] = get_b(c0, s, c);
      if constexpr (NORM) {
        const u32x4_t gm = get_g(c0, s);
#pragma unroll
        for (int c = 0; c < MS; ++c) B[s][c] = rms_scale8<DT>(B[s][c], gm, rr[c]);
      }
    }
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += GB) {
      u32x4_t A[GB][CH];
#pragma unroll
      for (int gg = 0; gg < GB; ++gg)
#pragma unroll
        for (int s = 0; s < CH; ++s) A[gg][s] = get_a(c0, g0 + gg, s);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int gg = 0; gg < GB; ++gg)
#pragma unroll
        for (int s = 0; s < CH; ++s)
#pragma unroll
          for (int c = 0; c < MS; ++c) {
            acc[g0 + gg][c] = Mfma4<DT>::step(lo2(A[gg][s]), lo2(B[s][c]), acc[g0 + gg][c]);
            acc[g0 + gg][c] = Mfma4<DT>::step(hi2(A[gg][s]), hi2(B[s][c]), acc[g0 + gg][c]);
          }
    }
  };
  int c0 = w0;
  if constexpr (NORM) {
    // the first chunk from what the prologue requested
    if (c0 < w1) {
      run_chunk(
          c0,
          [&](int cc, int s, int c) {
            if constexpr (kPreB) return B0[s][c];
            else return load_b(cc, s, c);
          },
          [&](int cc, int s) {
            if constexpr (kPreB) return G0[s];
            else return load_g(cc, s);
          },
          [&](int, int g, int s) { return A0[g][s]; });
      c0 += CH;
    }
  }
  for (; c0 < w1; c0 += CH) run_chunk(c0, load_b, load_g, load_a);

  // sum the 16 k-chunk blocks (lane bits 2..5), then the KS waves in wave
  // order through LDS: red[wave][value][col j]
  constexpr int NV = G * MS * 4;
  float val[NV];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int c = 0; c < MS; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) val[(g * MS + c) * 4 + v] = acc[g][c][v];
  reduce_lanes<NV, 4>(val);   // the 16 k blocks: lane bits 2..5
  __shared__ float red[KS * NV * 4];
  if (((lane >> 2) & 3) == 0) {
    const int q0 = ((lane >> 5) & 1) * (NV / 2) + ((lane >> 4) & 1) * (NV / 4);
#pragma unroll
    for (int p = 0; p < NV / 4; ++p) red[(wk * NV + q0 + p) * 4 + i4] = val[p];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < (GLU ? G / 2 : G) * MS * 16; e += 64 * KS) {
    const int j = e & 3, v = (e >> 2) & 3, c = (e >> 4) % MS, g = (e >> 4) / MS;
    const int64_t n = n_tile + 4 * g + v;
    const int64_t m = m_tile + 4 * c + j;
    if (n < N && m < M) {
      float t = 0.f, u = 0.f;
      for (int w = 0; w < KS; ++w) t += red[((w * G + g) * MS + c) * 16 + v * 4 + j];
      if (GLU)
        for (int w = 0; w < KS; ++w) u += red[((w * G + g + G / 2) * MS + c) * 16 + v * 4 + j];
      put_out<DT, PARTIAL, GLU>(a, split_id, m, n, t, u);
    }
  }
}

// ---------------------------------------------------------------------------
// 9..32 tokens: v_mfma_f32_16x16x32 fed from contiguous weight loads (4 rows x
// 256 bytes per instruction, the GEMV's access pattern) through a per-wave LDS
// tile (accum_lds).  Activations are the B operand as in thin_gemm_kernel.
// OUTR > 0: tiles of OUTR < 16 RB weight rows (24 rows on two 16-row blocks,
// the second half-filled), so that N = 6144 gives 256 workgroups instead of
// 192 of 32 rows or 384 of 16.

template <int DT, int RB, int CB, int KS, int U, bool PARTIAL, bool GLU, int OUTR = 0>
__global__ __launch_bounds__(64 * KS) void thin_gemm_lds_kernel(const char* __restrict__ w, const char* __restrict__ x,
                                                                const char* __restrict__ w2, uint32_t Kb,
                                                                uint32_t swn_b, uint32_t sxm_b, uint32_t sw2n_b, int N,
                                                                int M, int steps, int steps_per_split, ThinArgs a) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  constexpr int NF = RB * CB;
  constexpr int ROWS = 16 * RB;
  static_assert(!GLU || RB == 2, "gated: block 0 = gate rows, block 1 = the same rows of up");
  static_assert(OUTR == 0 || (!GLU && OUTR % 4 == 0 && OUTR > 16 * (RB - 1) && OUTR < ROWS),
                "partial tiles: ungated, whole 4-row groups, the last block part-filled");
  constexpr int OUT = GLU ? 16 : (OUTR > 0 ? OUTR : ROWS);   // output columns per workgroup
  // the waves' LDS tiles, reused for the cross-wave reduction once all waves
  // are past their main loop
  constexpr int kTileRows = ROWS + (SIMSD_LDS_X ? 16 * CB : 0);
  constexpr int kTileBytes = KS * kTileRows * kLdsRow;
  constexpr int kRedBytes = (KS > 1 ? (KS - 1) * NF * 4 * 64 : 1) * 4;
  static_assert(kTileBytes <= kLdsBytesGfx950 && kRedBytes <= kLdsBytesGfx950,
                "LDS tiles beyond gfx950's 160 KiB per workgroup");
  __shared__ __attribute__((aligned(16))) char smem[kTileBytes > kRedBytes ? kTileBytes : kRedBytes];
  const int lane = threadIdx.x & 63;
  const int wk = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int64_t n_tile = (int64_t)blockIdx.x * OUT;
  const int64_t m_tile = (int64_t)blockIdx.z * (CB * 16);
  const int split_id = blockIdx.y;

  // chunks of 256 B per row (4 MFMA k-steps) of this workgroup, then of this wave
  const int s_lo = split_id * steps_per_split;
  const int s_hi = min(steps, s_lo + steps_per_split);
  const int span = max(0, s_hi - s_lo);
  const int per_w = (span + KS - 1) / KS;
  const int w0 = s_lo + wk * per_w;
  const int w1 = min(s_hi, w0 + per_w);

  const int64_t rows_valid = min((int64_t)OUT, (int64_t)N - n_tile);
  const int64_t cols_valid = min((int64_t)(CB * 16), (int64_t)M - m_tile);
  const rsrc_t rA = make_rsrc(w + n_tile * swn_b, (uint32_t)(rows_valid - 1) * swn_b + Kb);
  const rsrc_t rB = make_rsrc(x + m_tile * sxm_b, (uint32_t)(cols_valid - 1) * sxm_b + Kb);
  f32x4_t acc[RB][CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  rsrc_t ra[RB];
  uint32_t a_row0[RB], a_sn[RB], boff[CB];
  bool bok[CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    ra[rb] = rA;
    a_row0[rb] = (uint32_t)(16 * rb) * swn_b;
    a_sn[rb] = swn_b;
  }
  if (GLU) {
    ra[RB - 1] = make_rsrc(w2 + n_tile * sw2n_b, (uint32_t)(rows_valid - 1) * sw2n_b + Kb);
    a_row0[RB - 1] = 0u;
    a_sn[RB - 1] = sw2n_b;
  }
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    boff[cb] = (uint32_t)(cb * 16 + r) * sxm_b;
    bok[cb] = cb * 16 + r < cols_valid;
  }
  if (SIMSD_LDS_X)
    accum_lds_ab<DT, RB, CB, U, GLU ? ROWS : OUT>(ra, a_row0, a_sn, rB, sxm_b, (int)cols_valid, w0, w1, Kb,
                                                  smem + wk * kTileRows * kLdsRow, acc);
  else
    accum_lds<DT, RB, CB, U, GLU ? ROWS : OUT>(ra, a_row0, a_sn, rB, boff, bok, w0, w1, Kb,
                                               smem + wk * kTileRows * kLdsRow, acc);

  __syncthreads();   // every wave done with its tile before the partials overwrite it
  reduce_waves<KS, NF>(reinterpret_cast<f32x4_t(&)[NF]>(acc), wk, lane, reinterpret_cast<float*>(smem));
  if (wk != 0) return;
#pragma unroll
  for (int rb = 0; rb < (GLU ? 1 : RB); ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int64_t m = m_tile + cb * 16 + r;
      const int64_t nb = n_tile + rb * 16 + 4 * g;
      if (m < M) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t n = nb + j;
          if (n < N && (OUTR == 0 || rb * 16 + 4 * g + j < OUT))
            put_out<DT, PARTIAL, GLU>(a, split_id, m, n, acc[rb][cb][j], acc[RB - 1][cb][j]);
        }
      }
    }
}

// ---------------------------------------------------------------------------
// 9..32 tokens, wide row tiles: the waves of a workgroup split its weight rows
// (wave w owns rows [16 RB w, 16 RB (w + 1)) of the tile, or, gated, 16 gate
// rows and the same 16 up rows) instead of K, so every wave needs the same
// activation chunk.  The workgroup loads each batch of U 256-byte activation
// chunks once -- its waves share the load instructions -- into one of two LDS
// slots, and all waves read their B operands from it; one barrier per batch
// (the double buffer makes the slot written next one that every wave has
// finished reading).  Each wave's weight chunks go through its own LDS tile as
// in accum_lds.  Activation bytes from L2 per weight byte: CB * 16 / (16 RB KS)
// instead of CB * 16 / (16 RB) -- a quarter at 128 rows.  No cross-wave sum:
// each wave writes its own outputs.
template <int DT, int RB, int CB, int KS, int U, bool PARTIAL, bool GLU>
__global__ __launch_bounds__(64 * KS) void thin_gemm_xs_kernel(const char* __restrict__ w, const char* __restrict__ x,
                                                               const char* __restrict__ w2, uint32_t Kb,
                                                               uint32_t swn_b, uint32_t sxm_b, uint32_t sw2n_b, int N,
                                                               int M, int steps, int steps_per_split, ThinArgs a) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  static_assert(!GLU || RB == 2, "gated: block 0 = gate rows, block 1 = the same rows of up");
  constexpr int WROWS = 16 * RB;                  // weight rows per wave
  constexpr int WOUT = GLU ? 16 : WROWS;          // output columns per wave
  constexpr int XROWS = 16 * CB;                  // activation rows (tokens) per tile
  constexpr int kXLoads = U * CB * 4;             // 4-row load instructions per activation batch
  constexpr int kXPer = (kXLoads + KS - 1) / KS;  // ... per wave
  constexpr int kSlot = U * XROWS * kLdsRow;
  static_assert(2 * kSlot + KS * WROWS * kLdsRow <= kLdsBytesGfx950,
                "shared-activation tile: LDS beyond gfx950's 160 KiB per workgroup (RB=2, CB=2, KS=4 "
                "takes 68 KiB, so these tiles need gfx950)");
  __shared__ __attribute__((aligned(16))) char xs[2 * kSlot];
  __shared__ __attribute__((aligned(16))) char wt[KS * WROWS * kLdsRow];
  const int lane = threadIdx.x & 63;
  // wave-uniform (the weight descriptors depend on it: a per-lane value would
  // put every buffer load in a readfirstlane loop)
  const int wk = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int g = lane >> 4, r = lane & 15;       // MFMA operand layout
  const int lr = lane >> 4, lc = lane & 15;     // loader layout: row l/16 of 4, chunk l%16
  const int64_t n_tile = (int64_t)blockIdx.x * (KS * WOUT);
  const int64_t n_wave = n_tile + (int64_t)wk * WOUT;
  const int64_t m_tile = (int64_t)blockIdx.z * XROWS;
  const int split_id = blockIdx.y;
  const int c0 = split_id * steps_per_split;
  const int c1 = min(steps, c0 + steps_per_split);

  // a wave past N keeps loading (zeros) and meeting the barriers
  const int64_t rows_w = max((int64_t)0, min((int64_t)WOUT, (int64_t)N - n_wave));
  const int64_t cols_valid = min((int64_t)XROWS, (int64_t)M - m_tile);
  rsrc_t ra[RB];
  uint32_t a_row0[RB], a_sn[RB];
  {
    const rsrc_t rw = make_rsrc(w + (rows_w > 0 ? n_wave * swn_b : 0),
                                rows_w > 0 ? (uint32_t)(rows_w - 1) * swn_b + Kb : 0u);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      ra[rb] = rw;
      a_row0[rb] = (uint32_t)(16 * rb) * swn_b;
      a_sn[rb] = swn_b;
    }
    if (GLU) {
      ra[RB - 1] = make_rsrc(w2 + (rows_w > 0 ? n_wave * sw2n_b : 0),
                             rows_w > 0 ? (uint32_t)(rows_w - 1) * sw2n_b + Kb : 0u);
      a_row0[RB - 1] = 0u;
      a_sn[RB - 1] = sw2n_b;
    }
  }
  const rsrc_t rx = make_rsrc(x + m_tile * sxm_b, (uint32_t)(cols_valid - 1) * sxm_b + Kb);
  f32x4_t acc[RB][CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  char* tile = wt + wk * WROWS * kLdsRow;
  // one batch: U chunks of this wave's weight rows and this wave's share of
  // the activation load instructions
  struct Batch {
    u32x4_t W[U][RB][4];
    u32x4_t X[kXPer];
  };
  // Past c1 every offset is out of range (zeros, no traffic).  The activation
  // loads go first: put_x then waits for them alone, with the weights still
  // in flight.
  auto load = [&](Batch& b, int c) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int li = wk + i * KS;   // this wave's i-th activation load instruction
      const int u = li / (CB * 4), row = (li % (CB * 4)) * 4 + lr;
      const uint32_t k = (uint32_t)(c + u) * kStep4Bytes + lc * kLaneBytes;
      const bool ok = li < kXLoads && c + u < c1 && k < Kb && row < cols_valid;
      b.X[i] = buf_load16<kAuxKeep>(rx, ok ? (uint32_t)row * sxm_b + k : kOob);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t k = (uint32_t)(c + u) * kStep4Bytes + lc * kLaneBytes;
      const bool kok = c + u < c1 && k < Kb;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          b.W[u][rb][q] = buf_load16<kAuxStream>(
              ra[rb], kok ? a_row0[rb] + (uint32_t)(4 * q + lr) * a_sn[rb] + k : kOob);
    }
  };
  auto put_x = [&](const Batch& b, char* xslot) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int li = wk + i * KS;
      if (li < kXLoads) {
        const int u = li / (CB * 4), row = (li % (CB * 4)) * 4 + lr;
        *reinterpret_cast<u32x4_t*>(xslot + (u * XROWS + row) * kLdsRow + lc * kLaneBytes) = b.X[i];
      }
    }
  };
  auto compute = [&](const Batch& b, const char* xslot) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<u32x4_t*>(tile + (16 * rb + 4 * q + lr) * kLdsRow + lc * kLaneBytes) = b.W[u][rb][q];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x4_t A[RB], B[CB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          A[rb] = *reinterpret_cast<const u32x4_t*>(tile + (16 * rb + r) * kLdsRow + j * kStepBytes +
                                                    g * kLaneBytes);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          B[cb] = *reinterpret_cast<const u32x4_t*>(xslot + (u * XROWS + 16 * cb + r) * kLdsRow +
                                                    j * kStepBytes + g * kLaneBytes);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = Mfma<DT>::step(A[rb], B[cb], acc[rb][cb]);
      }
    }
  };
  // Two batches in registers, used in turn: the next batch's loads are issued
  // after the barrier that publishes this batch's activations and before its
  // arithmetic, so they are in flight through the arithmetic and the next
  // barrier.  The loop is unrolled by hand over the two buffers.
  if (c0 < c1) {
    Batch bA, bB;
    load(bA, c0);
    for (int c = c0;;) {
      put_x(bA, xs);
      lds_barrier();   // batch c's activations are in slot 0
      load(bB, c + U);
      compute(bA, xs);
      c += U;
      if (c >= c1) break;
      put_x(bB, xs + kSlot);
      lds_barrier();   // slot 1
      load(bA, c + U);
      compute(bB, xs + kSlot);
      c += U;
      if (c >= c1) break;
    }
  }
  if (rows_w == 0) return;
#pragma unroll
  for (int rb = 0; rb < (GLU ? 1 : RB); ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int64_t m = m_tile + cb * 16 + r;
      const int64_t nb = n_wave + rb * 16 + 4 * g;
      if (m < M) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t n = nb + j;
          if (n < N) put_out<DT, PARTIAL, GLU>(a, split_id, m, n, acc[rb][cb][j], acc[RB - 1][cb][j]);
        }
      }
    }
}

// ---------------------------------------------------------------------------
// RMSNorm, one workgroup per token row: y = dtype(gamma * dtype(x * r)),
// r = 1 / sqrt(sum(x^2) / K + eps) in fp32 -- the stock PyTorch RMSNorm
// (sdar/run_native_tp2.py:42-47).  Sum order fixed (strided per thread, then
// waves in order): bit-reproducible.
template <int DT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const char* __restrict__ x, int64_t sxm,
                                                      const char* __restrict__ gamma, float eps,
                                                      char* __restrict__ y, int64_t sym, int64_t K) {
  __shared__ float part[4];
  const int64_t m = blockIdx.x;
  const char* xr = x + m * sxm * DTypeInfo<DT>::kSize;
  float acc = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const float v = load_elem<DT>(xr, k);
    acc += v * v;
  }
  const float t = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = t;
  __syncthreads();
  const float r = 1.f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)K + eps);
  char* yr = y + m * sym * DTypeInfo<DT>::kSize;
  for (int64_t k = threadIdx.x; k < K; k += 256)
    store_elem<DT>(yr, k, load_elem<DT>(gamma, k) * round_to<DT>(load_elem<DT>(xr, k) * r));
}

// 16-bit rows with K % 8 == 0 and K <= R * 2048, 16-byte aligned: the 256
// threads hold the row and gamma in registers (R 16-byte chunks each), so x
// and gamma are requested once, up front, and the row is read only once.
constexpr int kNormVecChunk = 256 * 8;   // elements per pass of the workgroup

template <int DT, int R>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const char* __restrict__ x, int64_t sxm,
                                                          const char* __restrict__ gamma, float eps,
                                                          char* __restrict__ y, int64_t sym, int64_t K) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  __shared__ float part[4];
  const int64_t m = blockIdx.x;
  const uint32_t Kb = (uint32_t)(K * ES);
  const rsrc_t rX = make_rsrc(x + m * sxm * ES, Kb);
  const rsrc_t rG = make_rsrc(gamma, Kb);
  u32x4_t v[R], g[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t off = (uint32_t)(i * 256 + threadIdx.x) * kLaneBytes;
    v[i] = buf_load16<kAuxKeep>(rX, off < Kb ? off : kOob);
    g[i] = buf_load16<kAuxKeep>(rG, off < Kb ? off : kOob);
  }
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i) acc = sumsq8<DT>(v[i], acc);
  const float t = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = t;
  __syncthreads();
  const float r = 1.f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)K + eps);
  char* yr = y + m * sym * ES;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t off = (uint32_t)(i * 256 + threadIdx.x) * kLaneBytes;
    if (off < Kb) *reinterpret_cast<u32x4_t*>(yr + off) = rms_scale8<DT>(v[i], g[i], r);
  }
}

// Sum the split partials in split order (fixed: bit-reproducible), round to
// the output dtype, add bias in the dtype.  One thread per output element.
template <int DT>
__global__ __launch_bounds__(256) void thin_reduce_kernel(const float* __restrict__ part, int split,
                                                          int64_t M, int64_t N,
                                                          const char* bias, int64_t sb, char* y,
                                                          int64_t sym, int64_t syn, int glu, const char* res,
                                                          int64_t srm, int64_t srn) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= M * N) return;
  const int64_t m = e / N, n = e % N;
  if (glu) {   // partial rows hold g in [0, N) and u in [N, 2N)
    float g = 0.f, u = 0.f;
    for (int s = 0; s < split; ++s) {
      const float* row = part + ((int64_t)s * M + m) * 2 * N;
      g += row[n];
      u += row[N + n];
    }
    store_elem<DT>(y, m * sym + n * syn, silu_mul<DT>(g, u));
    return;
  }
  float v = 0.f;
  for (int s = 0; s < split; ++s) v += part[(int64_t)s * M * N + e];
  if (bias != nullptr) v = round_to<DT>(v) + load_elem<DT>(bias, n * sb);
  if (res != nullptr) v = round_to<DT>(v) + load_elem<DT>(res, m * srm + n * srn);
  store_elem<DT>(y, m * sym + n * syn, v);
}

// A projection's split-K partials consumed by the residual add and the next
// RMSNorm, one workgroup per token row: h = dtype(dtype(sum) + res) (the
// partials summed in split order, the dtype's residual add), written to the
// residual stream, then xn = dtype(gamma * dtype(h * r)) with
// r = 1 / sqrt(sum(h^2) / N + eps) -- what thin_reduce_kernel followed by
// rmsnorm_vec_kernel compute, with the same element orders, so the results
// are bit-identical, in one launch.  16-bit rows, N % 8 == 0, N <= R * 2048,
// P >= split partials (loads past split are answered by the range check and
// dropped by selects, so none waits behind a branch).  res may alias h: each
// element is read before the same thread writes it.
constexpr int kReduceNormMaxSplit = 8;   // partials a consuming norm launch sums

template <int DT, int R, int P>
__global__ __launch_bounds__(256) void reduce_residual_rmsnorm_kernel(
    const float* __restrict__ part, int split, uint32_t part_split_bytes, const char* res, int64_t srm, char* h,
    int64_t shm, const char* __restrict__ gamma, float eps, char* __restrict__ xn, int64_t sxn, int64_t N) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  __shared__ float wsum[4];
  const int64_t m = blockIdx.x;
  const uint32_t Nb = (uint32_t)(N * ES);
  const rsrc_t rP = make_rsrc(part + m * N, (uint32_t)(split - 1) * part_split_bytes + (uint32_t)(N * 4));
  const rsrc_t rR = make_rsrc(res + m * srm * ES, Nb);
  const rsrc_t rG = make_rsrc(gamma, Nb);
  u32x4_t pv[R][P][2], rv[R], gv[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t e = (uint32_t)(i * 256 + threadIdx.x) * 8;   // first element of this lane's 8
    const bool ok = e * ES < Nb;
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const uint32_t o = (uint32_t)s * part_split_bytes + e * 4;
      pv[i][s][0] = buf_load16<kAuxKeep>(rP, ok && s < split ? o : kOob);
      pv[i][s][1] = buf_load16<kAuxKeep>(rP, ok && s < split ? o + 16 : kOob);
    }
    rv[i] = buf_load16<kAuxKeep>(rR, ok ? e * ES : kOob);
    gv[i] = buf_load16<kAuxKeep>(rG, ok ? e * ES : kOob);
  }
  u32x4_t hv[R];
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t rw[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {   // elements 2q, 2q + 1
      float v[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int el = 2 * q + j;
        const u32x4_t& c0 = pv[i][0][el >> 2];
        const uint32_t b0 = (el & 3) == 0 ? c0.x : (el & 3) == 1 ? c0.y : (el & 3) == 2 ? c0.z : c0.w;
        float t = __uint_as_float(b0);
        if (split > 1) t = 0.f + t;   // thin_reduce_kernel's sum starts from 0
#pragma unroll
        for (int s = 1; s < P; ++s) {
          const u32x4_t& cs = pv[i][s][el >> 2];
          const uint32_t bs = (el & 3) == 0 ? cs.x : (el & 3) == 1 ? cs.y : (el & 3) == 2 ? cs.z : cs.w;
          t = s < split ? t + __uint_as_float(bs) : t;
        }
        v[j] = round_to<DT>(round_to<DT>(t) + h16_to_f32<DT>(rw[q] >> (16 * j)));
      }
      o[q] = f32_to_h16<DT>(v[0]) | (f32_to_h16<DT>(v[1]) << 16);
    }
    hv[i] = u32x4_t{o[0], o[1], o[2], o[3]};
    acc = sumsq8<DT>(hv[i], acc);
  }
  const float t = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = t;
  __syncthreads();
  const float r = 1.f / sqrtf((wsum[0] + wsum[1] + wsum[2] + wsum[3]) / (float)N + eps);
  char* hr = h + m * shm * ES;
  char* yr = xn + m * sxn * ES;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t off = (uint32_t)(i * 256 + threadIdx.x) * 8 * ES;
    if (off < Nb) {
      *reinterpret_cast<u32x4_t*>(hr + off) = hv[i];
      *reinterpret_cast<u32x4_t*>(yr + off) = rms_scale8<DT>(hv[i], gv[i], r);
    }
  }
}

// ------------------------------------------------------------------ host side
namespace {

// kind 0: thin_gemm_kernel (16x16 MFMA; fp32 and strided views)
// kind 1: thin_gemv4_kernel (4x4x4 MFMA; M <= 8, bf16/fp16, vector-capable)
// kind 2: thin_gemm_lds_kernel (16x16x32 MFMA via LDS; M > 8, bf16/fp16, vector-capable)
struct ThinPlan {
  int kind;
  bool glu;                  // gated: rows are half gate, half up; outputs = rows / 2
  bool norm;                 // RMSNorm prologue in the GEMV
  int rows, rt, rb, cb, ms, ks, ch, split;
  bool fast;
  bool part_out;             // fp32 partials to the caller (even at split 1), no reduce launch
  int64_t tiles_n, tiles_m;
  int steps, steps_per_split;
  int64_t part_bytes;
};

inline int esize_of(int dtype) { return dtype == kF32 ? 4 : 2; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr int kMinWorkgroups = 256;   // one per CU on MI355X
constexpr int kMaxSplit = 16;

inline int fast_kind(int64_t M, int dtype) { return dtype == kF32 ? 0 : (M <= 8 ? 1 : 2); }

// the RMSNorm prologue runs inside the GEMV (else: norm launch, plain linear)
inline bool norm_in_gemv(const ThinPlan& pl, int64_t M, int64_t K, int es) {
  return pl.fast && pl.kind == 1 && pl.ms <= kNormMaxMs &&
         pl.tiles_n * pl.split * M * K * es <= SIMSD_NORM_STATS_BUDGET;
}

// Geometry only (no pointers).  block_n = weight rows per workgroup (0 = the
// most of 16, 8, 4 that still gives every CU a workgroup); split along K only
// when even 4-row tiles leave more than half the CUs idle (0 = automatic),
// keeping at least 256 bytes of every row per wave and split.
int plan_geometry(ThinPlan& pl, int kind, int64_t M, int64_t N, int64_t K, int dtype, int block_n,
                  int block_k, int num_waves, int split_k, bool glu = false) {
  const int es = esize_of(dtype);
  if (N > 0x7fffffff || M > 0x7fffffff)   // the GEMV takes them as 32-bit kernel arguments
    return set_error("thin_linear: N=%lld and M=%lld must be below 2^31", (long long)N, (long long)M);
  pl.kind = kind;
  pl.glu = glu;
  // GEMV activations held per chunk: 256 (2 load steps) or 1024 (8) k elements
  pl.ch = block_k >= 512 ? 8 : 2;
  // MFMA column blocks of 16 tokens: one up to 16, two up to 32; the 16-bit
  // LDS-staged kernels also take three (33..48 tokens in one pass over the
  // weight: the target's verify rows with a committed prefix folded in);
  // more tokens go in 32-token tiles
  pl.cb = M <= 16 ? 1 : ((kind == 2 && M > 32 && M <= 48) ? 3 : 2);
  pl.ms = M <= 4 ? 1 : 2;
  pl.tiles_m = kind == 1 ? cdiv(M, 4 * pl.ms) : cdiv(M, 16 * pl.cb);
  pl.ks = num_waves <= 0 ? 4 : num_waves;
  if (pl.ks != 2 && pl.ks != 4 && pl.ks != 8)
    return set_error("thin_linear: num_waves must be 2, 4 or 8 (got %d)", num_waves);
  int rows = block_n;
  if (rows == 0) {
    rows = 4;
    for (int cand : {16, 8}) {
      if (cdiv(N, cand) * pl.tiles_m >= kMinWorkgroups) { rows = cand; break; }
    }
  }
  if (rows != 4 && rows != 8 && rows != 16 && rows != 24 && rows != 32 && rows != 64 && rows != 96 &&
      rows != 128)
    return set_error("thin_linear: block_n must be 4, 8, 16, 24, 32, 64, 96 or 128 (got %d)", block_n);
  if (rows > 32 && kind != 2) rows = 32;   // 64, 96, 128: the 9..32-token kernel's shared-activation tiles
  if (rows == 24 && (kind != 2 || glu)) rows = 16;   // 24: the ungated 9..32-token kernel only
  if (kind == 2 && rows < 16) rows = 16;   // whole 16-row MFMA blocks
  if (glu && kind == 1 && rows < 8) rows = 8;    // gated GEMV: a gate and an up row group
  if (glu && kind == 2 && rows < 64) rows = 32;  // gated LDS kernel: a gate and an up block
  pl.rows = rows;
  pl.rt = rows >= 16 ? 16 : rows;
  pl.rb = rows >= 16 ? (rows + 15) / 16 : 1;
  if (kind == 2 && rows > 32) {
    // thin_gemm_xs_kernel: the waves split the rows, 16 or 32 each (gated: 32,
    // a gate and an up block); wave counts that do not divide the rows that
    // way take 32 rows per wave (96 rows: always 3 waves of 32)
    pl.kind = 3;
    pl.rb = rows % (16 * pl.ks) == 0 ? rows / (16 * pl.ks) : 0;
    if (pl.rb < 1 || pl.rb > 2 || (glu && pl.rb != 2)) {
      pl.rb = 2;
      pl.ks = rows / 32;
    }
  }
  // 48 tokens on two 16-row blocks: 8 waves' LDS tiles would pass gfx950's
  // 160 KiB, so such plans take 4 waves
  if (pl.kind == 2 && pl.cb == 3 && pl.rb == 2 && pl.ks == 8) pl.ks = 4;
  pl.tiles_n = cdiv(N, rows);
  pl.steps = (int)cdiv(K * es, kind == 0 ? kStepBytes : kStep4Bytes);
  int split = split_k;
  if (split <= 0) {
    const int64_t wgs = pl.tiles_n * pl.tiles_m;
    split = 1;
    if (wgs > 0 && wgs < kMinWorkgroups / 2) {   // wgs == 0: an empty M or N, nothing to split
      split = (int)cdiv(kMinWorkgroups, wgs);
      const int64_t max_by_k = (K * es) / (kStep4Bytes * (int64_t)pl.ks);
      split = (int)max((int64_t)1, min((int64_t)min(split, kMaxSplit), max_by_k));
    }
  }
  if (split > 1024) return set_error("thin_linear: split_k=%d exceeds 1024", split);
  pl.split = split;
  pl.steps_per_split = (int)cdiv(pl.steps, split);
  pl.part_bytes = split > 1 ? (int64_t)split * M * N * 4 : 0;
  return 0;
}

int make_plan(ThinPlan& pl, const void* x, int64_t sxm, int64_t sxk, const void* w, int64_t swn,
              int64_t swk, int64_t M, int64_t N, int64_t K, int dtype, int block_n, int block_k,
              int split_k, int num_waves, bool glu = false) {
  const int es = esize_of(dtype);
  const bool w_vec = swk == 1 && aligned16(w) && ((swn * es) % 16 == 0 || N == 1) &&
                     (K * es) % 16 == 0;
  const bool x_vec = sxk == 1 && aligned16(x) && ((sxm * es) % 16 == 0 || M == 1);
  // buffer descriptors address a tile with 32-bit offsets (a single row's
  // stride is never used)
  const int64_t w_extent = (N > 1 ? 31 * swn * es : 0) + K * es;
  const int64_t x_extent = (M > 1 ? 31 * sxm * es : 0) + K * es;
  const bool fast = w_vec && x_vec && (N == 1 || swn > 0) && (M == 1 || sxm > 0) &&
                    w_extent < (int64_t)kOob && x_extent < (int64_t)kOob;
  // The strided path has one shape: 16 rows per workgroup, 4 waves.
  if (plan_geometry(pl, fast ? fast_kind(M, dtype) : 0, M, N, K, dtype, fast ? block_n : 16,
                    block_k, fast ? num_waves : 4, split_k, glu) != 0)
    return -1;
  pl.fast = fast;
  return 0;
}

// 16-byte loads, K-contiguous rows, 32-bit-addressable tiles: the operand
// conditions of the fast kernels for a second weight matrix.
bool weight_vec_ok(const void* w, int64_t swn, int64_t swk, int64_t N, int64_t K, int es) {
  return w != nullptr && swk == 1 && aligned16(w) && ((swn * es) % 16 == 0 || N == 1) &&
         (K * es) % 16 == 0 && (N == 1 || swn > 0) &&
         (N > 1 ? 31 * swn * es : 0) + K * es < (int64_t)kOob;
}

template <bool PARTIAL, typename Kern>
void launch(Kern k, const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  dim3 grid((unsigned)pl.tiles_n, (unsigned)pl.split, (unsigned)pl.tiles_m);
  hipLaunchKernelGGL(k, grid, dim3(64 * pl.ks), 0, stream, args);
}

// The vector-capable kernels (GEMV, LDS and shared-activation tiles) take the
// fields their first loads depend on as leading scalar arguments, which the
// build preloads into SGPRs, then ThinArgs for the rest.
template <int DT, typename Kern>
void launch_hot(Kern k, const ThinPlan& pl, const ThinArgs& a, hipStream_t stream) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  const dim3 grid((unsigned)pl.tiles_n, (unsigned)pl.split, (unsigned)pl.tiles_m);
  hipLaunchKernelGGL(k, grid, dim3(64 * pl.ks), 0, stream, a.w, a.x, a.w2, (uint32_t)(a.K * ES),
                     (uint32_t)(a.swn * ES), (uint32_t)(a.sxm * ES), (uint32_t)(a.sw2n * ES), (int)a.N, (int)a.M,
                     a.steps, a.steps_per_split, a);
}

template <int DT, int RT, int RB, int CB, int KS, bool FAST>
void launch_gemm(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  constexpr int U = (RB * CB == 1) ? SIMSD_THIN_U : SIMSD_THIN_U / 2;
  if (pl.split > 1 || pl.part_out) launch<true>(thin_gemm_kernel<DT, RT, RB, CB, KS, U, FAST, true>, pl, args, stream);
  else launch<false>(thin_gemm_kernel<DT, RT, RB, CB, KS, U, FAST, false>, pl, args, stream);
}

template <int DT, int RT, int RB, int CB>
void gemm_ks(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  switch (pl.ks) {
    case 2: launch_gemm<DT, RT, RB, CB, 2, true>(pl, args, stream); break;
    case 8: launch_gemm<DT, RT, RB, CB, 8, true>(pl, args, stream); break;
    default: launch_gemm<DT, RT, RB, CB, 4, true>(pl, args, stream); break;
  }
}

template <int DT, int CB>
void gemm_rows(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  if (!pl.fast) {   // strided path: one shape, 16 rows, 4 waves
    launch_gemm<DT, 16, 1, CB, 4, false>(pl, args, stream);
    return;
  }
  switch (pl.rows) {
    case 4: gemm_ks<DT, 4, 1, CB>(pl, args, stream); break;
    case 8: gemm_ks<DT, 8, 1, CB>(pl, args, stream); break;
    case 32: gemm_ks<DT, 16, 2, CB>(pl, args, stream); break;
    default: gemm_ks<DT, 16, 1, CB>(pl, args, stream); break;
  }
}

#ifndef SIMSD_GEMV_GB_ALL
#define SIMSD_GEMV_GB_ALL 0   // 1: every row group's loads of a chunk issued together
#endif
#ifndef SIMSD_GEMV_CH_BIG
#define SIMSD_GEMV_CH_BIG 8   // load steps per chunk for block_k >= 512
#endif

template <int DT, int RW, int MS, int KS, int CH, bool GLU, bool NORM>
void launch_gemv4_ch(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  // gated: each batch of row groups stays inside the gate half or the up half
  constexpr int G = RW / 4;
  constexpr int GB = GLU ? (SIMSD_GEMV_GB_ALL ? G / 2 : (G >= 4 ? 2 : 1))
                         : (SIMSD_GEMV_GB_ALL ? G : (RW >= 8 ? 2 : 1));
  if (pl.split > 1 || pl.part_out) launch_hot<DT>(thin_gemv4_kernel<DT, RW, MS, KS, CH, GB, true, GLU, NORM>, pl, args, stream);
  else launch_hot<DT>(thin_gemv4_kernel<DT, RW, MS, KS, CH, GB, false, GLU, NORM>, pl, args, stream);
}

// The big chunk holds CH x (row groups + token sets) operand registers; at 8
// waves (256 VGPRs a wave) with 16 or more rows, or 8 tokens, it would spill,
// so those shapes keep the small chunk whatever block_k asks for.
template <int RW, int MS, int KS>
constexpr bool kBigChunkFits = !(KS == 8 && (RW >= 16 || MS == 2));

template <int DT, int RW, int MS, int KS, bool GLU, bool NORM>
void launch_gemv4(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  if constexpr (kBigChunkFits<RW, MS, KS>) {
    if (pl.ch == 8) {
      launch_gemv4_ch<DT, RW, MS, KS, SIMSD_GEMV_CH_BIG, GLU, NORM>(pl, args, stream);
      return;
    }
  }
  launch_gemv4_ch<DT, RW, MS, KS, 2, GLU, NORM>(pl, args, stream);
}

template <int DT, int RW, int MS, bool GLU, bool NORM>
void gemv4_ks(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  switch (pl.ks) {
    case 2: launch_gemv4<DT, RW, MS, 2, GLU, NORM>(pl, args, stream); break;
    case 8: launch_gemv4<DT, RW, MS, 8, GLU, NORM>(pl, args, stream); break;
    default: launch_gemv4<DT, RW, MS, 4, GLU, NORM>(pl, args, stream); break;
  }
}

template <int DT, int MS, bool GLU, bool NORM = false>
void gemv4_rows(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  switch (pl.rows) {
    case 4:
      if constexpr (!GLU) gemv4_ks<DT, 4, MS, false, NORM>(pl, args, stream);   // gated plans use >= 8
      break;
    case 8: gemv4_ks<DT, 8, MS, GLU, NORM>(pl, args, stream); break;
    case 32: gemv4_ks<DT, 32, MS, GLU, NORM>(pl, args, stream); break;
    default: gemv4_ks<DT, 16, MS, GLU, NORM>(pl, args, stream); break;
  }
}

#ifndef SIMSD_LDS_U
#define SIMSD_LDS_U 4
#endif

template <int DT, int RB, int CB, int KS, bool GLU, int OUTR>
void launch_lds(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  constexpr int U = (RB * CB == 1) ? SIMSD_LDS_U : (SIMSD_LDS_U + 1) / 2;
  if (pl.split > 1 || pl.part_out) launch_hot<DT>(thin_gemm_lds_kernel<DT, RB, CB, KS, U, true, GLU, OUTR>, pl, args, stream);
  else launch_hot<DT>(thin_gemm_lds_kernel<DT, RB, CB, KS, U, false, GLU, OUTR>, pl, args, stream);
}

template <int DT, int RB, int CB, bool GLU = false, int OUTR = 0>
void lds_ks(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  // 8 waves of 32-row x 48-token tiles do not fit the LDS; their plans take 4
  constexpr bool kEightFit = !(RB == 2 && CB == 3);
  switch (pl.ks) {
    case 2: launch_lds<DT, RB, CB, 2, GLU, OUTR>(pl, args, stream); break;
    case 8:
      if constexpr (kEightFit) {
        launch_lds<DT, RB, CB, 8, GLU, OUTR>(pl, args, stream);
        break;
      }
      [[fallthrough]];
    default: launch_lds<DT, RB, CB, 4, GLU, OUTR>(pl, args, stream); break;
  }
}

#ifndef SIMSD_XS_U
#define SIMSD_XS_U 2
#endif

template <int DT, int RB, int CB, int KS, bool GLU>
void launch_xs(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  constexpr int U = SIMSD_XS_U;
  if (pl.split > 1 || pl.part_out) launch_hot<DT>(thin_gemm_xs_kernel<DT, RB, CB, KS, U, true, GLU>, pl, args, stream);
  else launch_hot<DT>(thin_gemm_xs_kernel<DT, RB, CB, KS, U, false, GLU>, pl, args, stream);
}

// (rb, ks) of a shared-activation plan: (2, 2), (2, 3), (2, 4); ungated also
// (1, 4), (1, 8)
template <int DT, int CB, bool GLU>
void xs_shape(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  if (pl.rb == 2) {
    if (pl.ks == 2) launch_xs<DT, 2, CB, 2, GLU>(pl, args, stream);
    else if (pl.ks == 3) launch_xs<DT, 2, CB, 3, GLU>(pl, args, stream);
    else launch_xs<DT, 2, CB, 4, GLU>(pl, args, stream);
  } else if constexpr (!GLU) {
    if (pl.ks == 4) launch_xs<DT, 1, CB, 4, false>(pl, args, stream);
    else launch_xs<DT, 1, CB, 8, false>(pl, args, stream);
  }
}

template <int DT>
void dispatch_dt(const ThinPlan& pl, const ThinArgs& args, hipStream_t stream) {
  if constexpr (DT != kF32) {
    if (pl.kind == 3) {
      if (pl.glu) {
        if (pl.cb == 1) xs_shape<DT, 1, true>(pl, args, stream);
        else if (pl.cb == 2) xs_shape<DT, 2, true>(pl, args, stream);
        else xs_shape<DT, 3, true>(pl, args, stream);
      } else {
        if (pl.cb == 1) xs_shape<DT, 1, false>(pl, args, stream);
        else if (pl.cb == 2) xs_shape<DT, 2, false>(pl, args, stream);
        else xs_shape<DT, 3, false>(pl, args, stream);
      }
    } else if (pl.norm) {   // RMSNorm prologue: GEMV plans only
      if (pl.glu) {
        if (pl.ms == 1) gemv4_rows<DT, 1, true, true>(pl, args, stream);
        else gemv4_rows<DT, 2, true, true>(pl, args, stream);
      } else {
        if (pl.ms == 1) gemv4_rows<DT, 1, false, true>(pl, args, stream);
        else gemv4_rows<DT, 2, false, true>(pl, args, stream);
      }
    } else if (pl.glu) {
      if (pl.kind == 1) {
        if (pl.ms == 1) gemv4_rows<DT, 1, true>(pl, args, stream);
        else gemv4_rows<DT, 2, true>(pl, args, stream);
      } else if (pl.cb == 1) {
        lds_ks<DT, 2, 1, true>(pl, args, stream);
      } else if (pl.cb == 2) {
        lds_ks<DT, 2, 2, true>(pl, args, stream);
      } else {
        lds_ks<DT, 2, 3, true>(pl, args, stream);
      }
    } else if (pl.kind == 1) {
      if (pl.ms == 1) gemv4_rows<DT, 1, false>(pl, args, stream);
      else gemv4_rows<DT, 2, false>(pl, args, stream);
    } else if (pl.kind == 2) {
      // 16-row blocks x 16-token blocks; 24 rows: two blocks, the second half-filled
      if (pl.cb == 1) {
        if (pl.rows == 32) lds_ks<DT, 2, 1>(pl, args, stream);
        else if (pl.rows == 24) lds_ks<DT, 2, 1, false, 24>(pl, args, stream);
        else lds_ks<DT, 1, 1>(pl, args, stream);
      } else if (pl.cb == 2) {
        if (pl.rows == 32) lds_ks<DT, 2, 2>(pl, args, stream);
        else if (pl.rows == 24) lds_ks<DT, 2, 2, false, 24>(pl, args, stream);
        else lds_ks<DT, 1, 2>(pl, args, stream);
      } else {
        if (pl.rows == 32) lds_ks<DT, 2, 3>(pl, args, stream);
        else if (pl.rows == 24) lds_ks<DT, 2, 3, false, 24>(pl, args, stream);
        else lds_ks<DT, 1, 3>(pl, args, stream);
      }
    }
  }
  if (pl.kind == 0) {
    if (pl.cb == 1) gemm_rows<DT, 1>(pl, args, stream);
    else gemm_rows<DT, 2>(pl, args, stream);
  }
  if (pl.split > 1 && !pl.part_out) {
    const int64_t total = args.M * args.N;
    hipLaunchKernelGGL((thin_reduce_kernel<DT>), dim3((unsigned)cdiv(total, 256)), dim3(256), 0,
                       stream, args.part, pl.split, args.M, args.N, args.bias, args.sb, args.y,
                       args.sym, args.syn, pl.glu ? 1 : 0, args.res, args.srm, args.srn);
  }
}

}  // namespace
}  // namespace simsd

using namespace simsd;

extern "C" int64_t simsd_thin_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int dtype,
                                                     int block_n, int split_k, int num_waves) {
  const int block_k = 0;   // the chunk size does not change the workspace
  // Enough for any path the call may take: either kernel with the requested
  // geometry, or the strided one (16 rows, 4 waves).
  ThinPlan a{}, b{}, c{};
  if (plan_geometry(a, 0, M, N, K, dtype, block_n, block_k, num_waves, split_k) != 0) return -1;
  if (plan_geometry(b, 0, M, N, K, dtype, 16, block_k, 4, split_k) != 0) return -1;
  if (plan_geometry(c, fast_kind(M, dtype), M, N, K, dtype, block_n, block_k, num_waves, split_k) != 0)
    return -1;
  int64_t need = a.part_bytes > b.part_bytes ? a.part_bytes : b.part_bytes;
  return need > c.part_bytes ? need : c.part_bytes;
}

extern "C" int simsd_thin_linear(const void* x, int64_t sxm, int64_t sxk, const void* w,
                                 int64_t swn, int64_t swk, const void* bias, int64_t sb, void* y,
                                 int64_t sym, int64_t syn, int64_t M, int64_t N, int64_t K,
                                 int dtype, int block_n, int block_k, int split_k, int num_waves,
                                 void* workspace, int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("thin_linear: unsupported dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return set_error("thin_linear: negative size");
  if (M == 0 || N == 0) return 0;
  if (K == 0) return set_error("thin_linear: K == 0 must be handled by the caller");
  if (x == nullptr || w == nullptr || y == nullptr) return set_error("thin_linear: null pointer");
  if (K * (int64_t)esize_of(dtype) > ((int64_t)1 << 31) - 64)
    return set_error("thin_linear: K=%lld too large", (long long)K);
  ThinPlan pl{};
  if (make_plan(pl, x, sxm, sxk, w, swn, swk, M, N, K, dtype, block_n, block_k, split_k, num_waves) != 0)
    return -1;
  if (pl.tiles_n > 0x7fffffff || pl.tiles_m > 65535 || cdiv(M * N, 256) > 0x7fffffff)
    return set_error("thin_linear: grid too large (N=%lld, M=%lld)", (long long)N, (long long)M);
  ThinArgs args{};
  args.x = static_cast<const char*>(x);
  args.sxm = sxm; args.sxk = sxk;
  args.w = static_cast<const char*>(w);
  args.swn = swn; args.swk = swk;
  args.bias = static_cast<const char*>(bias);
  args.sb = sb;
  args.y = static_cast<char*>(y);
  args.sym = sym; args.syn = syn;
  args.M = M; args.N = N; args.K = K;
  args.steps = pl.steps;
  args.steps_per_split = pl.steps_per_split;
  if (pl.split > 1) {
    if (workspace == nullptr || workspace_bytes < pl.part_bytes)
      return set_error("thin_linear: split_k=%d needs a %lld-byte workspace (got %lld)", pl.split,
                       (long long)pl.part_bytes, (long long)workspace_bytes);
    if (!aligned16(workspace)) return set_error("thin_linear: workspace must be 16-byte aligned");
    args.part = static_cast<float*>(workspace);
  }
  switch (dtype) {
    case kBF16: dispatch_dt<kBF16>(pl, args, stream); break;
    case kF16: dispatch_dt<kF16>(pl, args, stream); break;
    default: dispatch_dt<kF32>(pl, args, stream); break;
  }
  return check_launch("thin_linear");
}

// ---------------------------------------------------------- allocation-free
// simsd_thin_linear_noalloc keeps its split-K partials in this file-scope
// device array instead of a caller workspace: each GPU the library runs on
// holds its own copy until the process ends.  In host code the name is a
// host-side stand-in, not a device address; the per-device address comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address is passed to kernels.
constexpr int64_t kNoAllocScratchBytes = 8ll << 20;   // 8 MiB
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (looked up on its first use).
int scratch_on_current_device(void** out) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) return set_error("thin_linear_noalloc: hipGetDevice failed: %s", hipGetErrorString(ge));
  if (dev < 0 || dev >= kMaxDevices) return set_error("thin_linear_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error("thin_linear_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int64_t simsd_thin_linear_noalloc_max_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int simsd_thin_linear_noalloc(const void* x, int64_t sxm, int64_t sxk, const void* w,
                                         int64_t swn, int64_t swk, const void* bias, int64_t sb, void* y,
                                         int64_t sym, int64_t syn, int64_t M, int64_t N, int64_t K,
                                         int dtype, int block_n, int block_k, int split_k, int num_waves,
                                         void* stream) {
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("thin_linear_noalloc: unsupported dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return set_error("thin_linear_noalloc: negative size");
  if (M == 0 || N == 0) return 0;   // as simsd_thin_linear: nothing to compute
  const int64_t need = simsd_thin_linear_workspace_bytes(M, N, K, dtype, block_n, split_k, num_waves);
  if (need < 0) return -1;
  if (need > kNoAllocScratchBytes)
    return set_error("thin_linear_noalloc: this shape and split need %lld bytes of split-K scratch, "
                     "above the static maximum of %lld bytes (use simsd_thin_linear with a workspace)",
                     (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (scratch_on_current_device(&ws) != 0) return -1;
  return simsd_thin_linear(x, sxm, sxk, w, swn, swk, bias, sb, y, sym, syn, M, N, K, dtype, block_n,
                           block_k, split_k, num_waves, ws, kNoAllocScratchBytes, stream);
}

extern "C" int simsd_thin_linear_plan(int64_t M, int64_t N, int64_t K, int dtype, int block_n,
                                      int split_k, int num_waves, int* out4) {
  const int block_k = 0;
  // (rows per workgroup, columns per block, waves per workgroup, split) of the
  // geometry a vector-capable call takes; lets the Python side report it.
  ThinPlan pl{};
  if (plan_geometry(pl, fast_kind(M, dtype), M, N, K, dtype, block_n, block_k, num_waves, split_k) != 0)
    return -1;
  out4[0] = pl.rows;
  out4[1] = pl.kind == 1 ? 4 * pl.ms : 16 * pl.cb;
  out4[2] = pl.ks;
  out4[3] = pl.split;
  return 0;
}

extern "C" int simsd_thin_linear_silu_mul(const void* x, int64_t sxm, int64_t sxk, const void* w_gate,
                                          int64_t sgn, int64_t sgk, const void* w_up, int64_t sun,
                                          int64_t suk, void* h, int64_t shm, int64_t shn, int64_t M,
                                          int64_t I, int64_t K, int dtype, int block_n, int block_k,
                                          int split_k, int num_waves, void* workspace,
                                          int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16)
    return set_error("thin_linear_silu_mul: dtype must be bf16 or fp16 (got code %d)", dtype);
  if (M < 0 || I < 0 || K < 0) return set_error("thin_linear_silu_mul: negative size");
  if (M == 0 || I == 0) return 0;
  if (K == 0) return set_error("thin_linear_silu_mul: K == 0 must be handled by the caller");
  if (x == nullptr || w_gate == nullptr || w_up == nullptr || h == nullptr)
    return set_error("thin_linear_silu_mul: null pointer");
  const int es = esize_of(dtype);
  if (K * (int64_t)es > ((int64_t)1 << 31) - 64)
    return set_error("thin_linear_silu_mul: K=%lld too large", (long long)K);
  ThinPlan pl{};
  // planned as one linear over the 2I stacked gate and up rows
  if (make_plan(pl, x, sxm, sxk, w_gate, sgn, sgk, M, 2 * I, K, dtype, block_n, block_k, split_k,
                num_waves, true) != 0)
    return -1;
  if (!pl.fast || !weight_vec_ok(w_up, sun, suk, I, K, es))
    return set_error("thin_linear_silu_mul: needs 16-byte aligned, K-contiguous x, w_gate and w_up");
  if (pl.tiles_n > 0x7fffffff || pl.tiles_m > 65535 || cdiv(M * I, 256) > 0x7fffffff)
    return set_error("thin_linear_silu_mul: grid too large (I=%lld, M=%lld)", (long long)I, (long long)M);
  ThinArgs args{};
  args.x = static_cast<const char*>(x);
  args.sxm = sxm; args.sxk = sxk;
  args.w = static_cast<const char*>(w_gate);
  args.swn = sgn; args.swk = sgk;
  args.w2 = static_cast<const char*>(w_up);
  args.sw2n = sun;
  args.y = static_cast<char*>(h);
  args.sym = shm; args.syn = shn;
  args.M = M; args.N = I; args.K = K;
  args.steps = pl.steps;
  args.steps_per_split = pl.steps_per_split;
  if (pl.split > 1) {
    if (workspace == nullptr || workspace_bytes < pl.part_bytes)
      return set_error("thin_linear_silu_mul: split_k=%d needs a %lld-byte workspace (got %lld)",
                       pl.split, (long long)pl.part_bytes, (long long)workspace_bytes);
    if (!aligned16(workspace)) return set_error("thin_linear_silu_mul: workspace must be 16-byte aligned");
    args.part = static_cast<float*>(workspace);
  }
  if (dtype == kBF16) dispatch_dt<kBF16>(pl, args, stream);
  else dispatch_dt<kF16>(pl, args, stream);
  return check_launch("thin_linear_silu_mul");
}

namespace {
// Shared tail of the entry points: workspace check, dispatch, launch check.
int run_planned(ThinPlan& pl, ThinArgs& args, int dtype, void* workspace, int64_t workspace_bytes,
                hipStream_t stream, const char* what) {
  if (pl.tiles_n > 0x7fffffff || pl.tiles_m > 65535 || cdiv(args.M * args.N, 256) > 0x7fffffff)
    return set_error("%s: grid too large (N=%lld, M=%lld)", what, (long long)args.N, (long long)args.M);
  if (pl.split > 1) {
    if (workspace == nullptr || workspace_bytes < pl.part_bytes)
      return set_error("%s: split_k=%d needs a %lld-byte workspace (got %lld)", what, pl.split,
                       (long long)pl.part_bytes, (long long)workspace_bytes);
    if (!aligned16(workspace)) return set_error("%s: workspace must be 16-byte aligned", what);
    args.part = static_cast<float*>(workspace);
  }
  switch (dtype) {
    case kBF16: dispatch_dt<kBF16>(pl, args, stream); break;
    case kF16: dispatch_dt<kF16>(pl, args, stream); break;
    default: dispatch_dt<kF32>(pl, args, stream); break;
  }
  return check_launch(what);
}

int launch_rmsnorm(const void* x, int64_t sxm, const void* gamma, float eps, void* y, int64_t sym,
                   int64_t M, int64_t K, int dtype, hipStream_t stream) {
  const dim3 grid((unsigned)M), block(256);
  const char* xc = static_cast<const char*>(x);
  const char* gc = static_cast<const char*>(gamma);
  char* yc = static_cast<char*>(y);
  const int64_t es = esize_of(dtype);
  const bool vec = dtype != kF32 && K % 8 == 0 && K <= 4 * kNormVecChunk && aligned16(x) && aligned16(y) &&
                   aligned16(gamma) && (sxm * es) % 16 == 0 && (sym * es) % 16 == 0;
  if (vec) {
    const int R = (int)cdiv(K, kNormVecChunk);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, 0, stream, xc, sxm, gc, eps, yc, sym, K); };
    if (dtype == kBF16) {
      if (R == 1) go(rmsnorm_vec_kernel<kBF16, 1>);
      else if (R == 2) go(rmsnorm_vec_kernel<kBF16, 2>);
      else go(rmsnorm_vec_kernel<kBF16, 4>);
    } else {
      if (R == 1) go(rmsnorm_vec_kernel<kF16, 1>);
      else if (R == 2) go(rmsnorm_vec_kernel<kF16, 2>);
      else go(rmsnorm_vec_kernel<kF16, 4>);
    }
    return check_launch("rmsnorm");
  }
  switch (dtype) {
    case kBF16: hipLaunchKernelGGL(rmsnorm_kernel<kBF16>, grid, block, 0, stream, xc, sxm, gc, eps, yc, sym, K); break;
    case kF16: hipLaunchKernelGGL(rmsnorm_kernel<kF16>, grid, block, 0, stream, xc, sxm, gc, eps, yc, sym, K); break;
    default: hipLaunchKernelGGL(rmsnorm_kernel<kF32>, grid, block, 0, stream, xc, sxm, gc, eps, yc, sym, K); break;
  }
  return check_launch("rmsnorm");
}

inline int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }
}  // namespace

extern "C" int simsd_rmsnorm(const void* x, int64_t sxm, const void* gamma, float eps, void* y,
                             int64_t sym, int64_t M, int64_t K, int dtype, void* stream_) {
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("rmsnorm: unsupported dtype code %d", dtype);
  if (M < 0 || K <= 0 || M > 0x7fffffff) return set_error("rmsnorm: bad sizes M=%lld K=%lld", (long long)M, (long long)K);
  if (M == 0) return 0;
  if (x == nullptr || gamma == nullptr || y == nullptr) return set_error("rmsnorm: null pointer");
  return launch_rmsnorm(x, sxm, gamma, eps, y, sym, M, K, dtype, static_cast<hipStream_t>(stream_));
}

extern "C" int64_t simsd_rmsnorm_linear_workspace_bytes(int64_t M, int64_t N_rows, int64_t K, int dtype,
                                                        int block_n, int split_k, int num_waves) {
  const int64_t part = simsd_thin_linear_workspace_bytes(M, N_rows, K, dtype, block_n, split_k, num_waves);
  if (part < 0) return -1;
  if (M == 0 || N_rows == 0) return 0;   // the entry points return before using a workspace
  return align256(M * K * esize_of(dtype)) + part;
}

extern "C" int simsd_rmsnorm_thin_linear(const void* x, int64_t sxm, int64_t sxk, const void* gamma,
                                         float eps, const void* w, int64_t swn, int64_t swk,
                                         const void* bias, int64_t sb, void* y, int64_t sym, int64_t syn,
                                         int64_t M, int64_t N, int64_t K, int dtype, int block_n,
                                         int block_k, int split_k, int num_waves, void* workspace,
                                         int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("rmsnorm_thin_linear: unsupported dtype code %d", dtype);
  if (M < 0 || N < 0 || K <= 0) return set_error("rmsnorm_thin_linear: bad sizes");
  if (M == 0 || N == 0) return 0;
  if (x == nullptr || gamma == nullptr || w == nullptr || y == nullptr)
    return set_error("rmsnorm_thin_linear: null pointer");
  if (sxk != 1) return set_error("rmsnorm_thin_linear: x must be K-contiguous");
  const int es = esize_of(dtype);
  if (K * (int64_t)es > ((int64_t)1 << 31) - 64) return set_error("rmsnorm_thin_linear: K too large");
  const int64_t xn_bytes = align256(M * K * es);
  ThinPlan pl{};
  if (make_plan(pl, x, sxm, sxk, w, swn, swk, M, N, K, dtype, block_n, block_k, split_k, num_waves) != 0)
    return -1;
  ThinArgs args{};
  args.sxk = 1;
  args.w = static_cast<const char*>(w); args.swn = swn; args.swk = swk;
  args.bias = static_cast<const char*>(bias); args.sb = sb;
  args.y = static_cast<char*>(y); args.sym = sym; args.syn = syn;
  args.M = M; args.N = N; args.K = K;
  // the norm runs inside the GEMV (up to 8 tokens); the MFMA-tile kernels
  // above take the normalised rows from a separate launch
  if (norm_in_gemv(pl, M, K, es) && aligned16(gamma)) {
    pl.norm = true;
    args.x = static_cast<const char*>(x); args.sxm = sxm;
    args.gamma = static_cast<const char*>(gamma); args.eps = eps;
    args.steps = pl.steps; args.steps_per_split = pl.steps_per_split;
    return run_planned(pl, args, dtype, workspace, workspace_bytes, stream, "rmsnorm_thin_linear");
  }
  // otherwise: normalise into the workspace, then the plain linear on it
  if (workspace == nullptr || workspace_bytes < xn_bytes || !aligned16(workspace))
    return set_error("rmsnorm_thin_linear: needs a 16-byte aligned workspace of at least %lld bytes",
                     (long long)xn_bytes);
  char* xn = static_cast<char*>(workspace);
  if (launch_rmsnorm(x, sxm, gamma, eps, xn, K, M, K, dtype, stream) != 0) return -1;
  if (make_plan(pl, xn, K, 1, w, swn, swk, M, N, K, dtype, block_n, block_k, split_k, num_waves) != 0)
    return -1;
  args.x = xn; args.sxm = K;
  args.steps = pl.steps; args.steps_per_split = pl.steps_per_split;
  return run_planned(pl, args, dtype, xn + xn_bytes, workspace_bytes - xn_bytes, stream,
                     "rmsnorm_thin_linear");
}

extern "C" int simsd_rmsnorm_thin_linear_silu_mul(const void* x, int64_t sxm, int64_t sxk,
                                                  const void* gamma, float eps, const void* w_gate,
                                                  int64_t sgn, int64_t sgk, const void* w_up, int64_t sun,
                                                  int64_t suk, void* h, int64_t shm, int64_t shn,
                                                  int64_t M, int64_t I, int64_t K, int dtype, int block_n,
                                                  int block_k, int split_k, int num_waves, void* workspace,
                                                  int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16)
    return set_error("rmsnorm_thin_linear_silu_mul: dtype must be bf16 or fp16 (got code %d)", dtype);
  if (M < 0 || I < 0 || K <= 0) return set_error("rmsnorm_thin_linear_silu_mul: bad sizes");
  if (M == 0 || I == 0) return 0;
  if (x == nullptr || gamma == nullptr || w_gate == nullptr || w_up == nullptr || h == nullptr)
    return set_error("rmsnorm_thin_linear_silu_mul: null pointer");
  if (sxk != 1) return set_error("rmsnorm_thin_linear_silu_mul: x must be K-contiguous");
  const int es = esize_of(dtype);
  if (K * (int64_t)es > ((int64_t)1 << 31) - 64) return set_error("rmsnorm_thin_linear_silu_mul: K too large");
  const int64_t xn_bytes = align256(M * K * es);
  ThinPlan pl{};
  if (make_plan(pl, x, sxm, sxk, w_gate, sgn, sgk, M, 2 * I, K, dtype, block_n, block_k, split_k,
                num_waves, true) != 0)
    return -1;
  if (!weight_vec_ok(w_up, sun, suk, I, K, es) || !weight_vec_ok(w_gate, sgn, sgk, I, K, es))
    return set_error("rmsnorm_thin_linear_silu_mul: needs 16-byte aligned, K-contiguous w_gate and w_up");
  ThinArgs args{};
  args.sxk = 1;
  args.w = static_cast<const char*>(w_gate); args.swn = sgn; args.swk = sgk;
  args.w2 = static_cast<const char*>(w_up); args.sw2n = sun;
  args.y = static_cast<char*>(h); args.sym = shm; args.syn = shn;
  args.M = M; args.N = I; args.K = K;
  if (norm_in_gemv(pl, M, K, es) && aligned16(gamma)) {
    pl.norm = true;
    args.x = static_cast<const char*>(x); args.sxm = sxm;
    args.gamma = static_cast<const char*>(gamma); args.eps = eps;
    args.steps = pl.steps; args.steps_per_split = pl.steps_per_split;
    return run_planned(pl, args, dtype, workspace, workspace_bytes, stream, "rmsnorm_thin_linear_silu_mul");
  }
  if (workspace == nullptr || workspace_bytes < xn_bytes || !aligned16(workspace))
    return set_error("rmsnorm_thin_linear_silu_mul: needs a 16-byte aligned workspace of at least %lld bytes",
                     (long long)xn_bytes);
  char* xn = static_cast<char*>(workspace);
  if (launch_rmsnorm(x, sxm, gamma, eps, xn, K, M, K, dtype, stream) != 0) return -1;
  if (make_plan(pl, xn, K, 1, w_gate, sgn, sgk, M, 2 * I, K, dtype, block_n, block_k, split_k, num_waves,
                true) != 0)
    return -1;
  if (!pl.fast) return set_error("rmsnorm_thin_linear_silu_mul: operands not vector-aligned");
  args.x = xn; args.sxm = K;
  args.steps = pl.steps; args.steps_per_split = pl.steps_per_split;
  return run_planned(pl, args, dtype, xn + xn_bytes, workspace_bytes - xn_bytes, stream,
                     "rmsnorm_thin_linear_silu_mul");
}

extern "C" int simsd_thin_linear_residual(const void* x, int64_t sxm, int64_t sxk, const void* w, int64_t swn,
                                          int64_t swk, const void* residual, int64_t srm, int64_t srn, void* y,
                                          int64_t sym, int64_t syn, int64_t M, int64_t N, int64_t K, int dtype,
                                          int block_n, int block_k, int split_k, int num_waves, void* workspace,
                                          int64_t workspace_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("thin_linear_residual: unsupported dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return set_error("thin_linear_residual: negative size");
  if (M == 0 || N == 0) return 0;
  if (K == 0) return set_error("thin_linear_residual: K == 0 must be handled by the caller");
  if (x == nullptr || w == nullptr || y == nullptr || residual == nullptr)
    return set_error("thin_linear_residual: null pointer");
  if (K * (int64_t)esize_of(dtype) > ((int64_t)1 << 31) - 64)
    return set_error("thin_linear_residual: K=%lld too large", (long long)K);
  ThinPlan pl{};
  if (make_plan(pl, x, sxm, sxk, w, swn, swk, M, N, K, dtype, block_n, block_k, split_k, num_waves) != 0)
    return -1;
  ThinArgs args{};
  args.x = static_cast<const char*>(x); args.sxm = sxm; args.sxk = sxk;
  args.w = static_cast<const char*>(w); args.swn = swn; args.swk = swk;
  args.y = static_cast<char*>(y); args.sym = sym; args.syn = syn;
  args.res = static_cast<const char*>(residual); args.srm = srm; args.srn = srn;
  args.M = M; args.N = N; args.K = K;
  args.steps = pl.steps; args.steps_per_split = pl.steps_per_split;
  return run_planned(pl, args, dtype, workspace, workspace_bytes, stream, "thin_linear_residual");
}


extern "C" int simsd_thin_linear_partials(const void* x, int64_t sxm, int64_t sxk, const void* w, int64_t swn,
                                          int64_t swk, void* part, int64_t part_bytes, int64_t M, int64_t N,
                                          int64_t K, int dtype, int block_n, int block_k, int split_k,
                                          int num_waves, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16 && dtype != kF32)
    return set_error("thin_linear_partials: unsupported dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return set_error("thin_linear_partials: negative size");
  if (split_k < 1 || split_k > kMaxSplit)
    return set_error("thin_linear_partials: split_k must be 1..%d (got %d)", kMaxSplit, split_k);
  if (M == 0 || N == 0) return 0;
  if (K == 0) return set_error("thin_linear_partials: K == 0 must be handled by the caller");
  if (x == nullptr || w == nullptr || part == nullptr) return set_error("thin_linear_partials: null pointer");
  if (!aligned16(part)) return set_error("thin_linear_partials: partials must be 16-byte aligned");
  if (K * (int64_t)esize_of(dtype) > ((int64_t)1 << 31) - 64)
    return set_error("thin_linear_partials: K=%lld too large", (long long)K);
  if (part_bytes < (int64_t)split_k * M * N * 4)
    return set_error("thin_linear_partials: %d partials of %lld x %lld need %lld bytes (got %lld)", split_k,
                     (long long)M, (long long)N, (long long)split_k * M * N * 4, (long long)part_bytes);
  ThinPlan pl{};
  if (make_plan(pl, x, sxm, sxk, w, swn, swk, M, N, K, dtype, block_n, block_k, split_k, num_waves) != 0)
    return -1;
  if (pl.split != split_k) return set_error("thin_linear_partials: plan split %d != %d", pl.split, split_k);
  if (pl.tiles_n > 0x7fffffff || pl.tiles_m > 65535)
    return set_error("thin_linear_partials: grid too large (N=%lld, M=%lld)", (long long)N, (long long)M);
  pl.part_out = true;
  ThinArgs args{};
  args.x = static_cast<const char*>(x); args.sxm = sxm; args.sxk = sxk;
  args.w = static_cast<const char*>(w); args.swn = swn; args.swk = swk;
  args.part = static_cast<float*>(part);
  args.M = M; args.N = N; args.K = K;
  args.steps = pl.steps; args.steps_per_split = pl.steps_per_split;
  switch (dtype) {
    case kBF16: dispatch_dt<kBF16>(pl, args, stream); break;
    case kF16: dispatch_dt<kF16>(pl, args, stream); break;
    default: dispatch_dt<kF32>(pl, args, stream); break;
  }
  return check_launch("thin_linear_partials");
}

extern "C" int simsd_reduce_residual_rmsnorm(const void* part, int split, int64_t part_bytes, const void* residual,
                                             int64_t srm, void* h, int64_t shm, const void* gamma, float eps,
                                             void* xn, int64_t sxn, int64_t M, int64_t N, int dtype, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (dtype != kBF16 && dtype != kF16) return set_error("reduce_residual_rmsnorm: dtype must be bf16 or fp16");
  if (M < 0 || N < 0) return set_error("reduce_residual_rmsnorm: negative size");
  if (split < 1 || split > kReduceNormMaxSplit)
    return set_error("reduce_residual_rmsnorm: split must be 1..%d (got %d)", kReduceNormMaxSplit, split);
  if (M == 0 || N == 0) return 0;
  if (N % 8 != 0 || N > 4 * kNormVecChunk)
    return set_error("reduce_residual_rmsnorm: N=%lld must be a multiple of 8 and at most %d", (long long)N,
                     4 * kNormVecChunk);
  if (!part || !residual || !h || !gamma || !xn) return set_error("reduce_residual_rmsnorm: null pointer");
  const int64_t es = 2;
  if (!aligned16(part) || !aligned16(residual) || !aligned16(h) || !aligned16(gamma) || !aligned16(xn) ||
      (srm * es) % 16 != 0 || (shm * es) % 16 != 0 || (sxn * es) % 16 != 0 || srm < N || shm < N || sxn < N)
    return set_error("reduce_residual_rmsnorm: 16-byte aligned rows of at least N elements required");
  const int64_t split_bytes = M * N * 4;
  if ((int64_t)split * split_bytes > part_bytes)
    return set_error("reduce_residual_rmsnorm: %d partials of %lld x %lld need %lld bytes (got %lld)", split,
                     (long long)M, (long long)N, (long long)split * split_bytes, (long long)part_bytes);
  if ((int64_t)split * split_bytes > (int64_t)0xFFFF0000)
    return set_error("reduce_residual_rmsnorm: partials past 32-bit offsets");
  const int R = (int)cdiv(N, kNormVecChunk);
  const float* pp = static_cast<const float*>(part);
  const char* rc = static_cast<const char*>(residual);
  char* hc = static_cast<char*>(h);
  const char* gc = static_cast<const char*>(gamma);
  char* yc = static_cast<char*>(xn);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)M), dim3(256), 0, stream, pp, split, (uint32_t)split_bytes, rc, srm,
                       hc, shm, gc, eps, yc, sxn, N);
  };
  auto by_p = [&](auto dt, auto r) {
    constexpr int DT = decltype(dt)::value, RR = decltype(r)::value;
    if (split == 1) go(reduce_residual_rmsnorm_kernel<DT, RR, 1>);
    else if (split == 2) go(reduce_residual_rmsnorm_kernel<DT, RR, 2>);
    else if (split <= 4) go(reduce_residual_rmsnorm_kernel<DT, RR, 4>);
    else go(reduce_residual_rmsnorm_kernel<DT, RR, 8>);
  };
  auto by_r = [&](auto dt) {
    if (R == 1) by_p(dt, std::integral_constant<int, 1>{});
    else if (R == 2) by_p(dt, std::integral_constant<int, 2>{});
    else by_p(dt, std::integral_constant<int, 4>{});
  };
  if (dtype == kBF16) by_r(std::integral_constant<int, kBF16>{});
  else by_r(std::integral_constant<int, kF16>{});
  return check_launch("reduce_residual_rmsnorm");
}

// Attention of a few query rows over a static KV cache, for the speculative
// step's draft blocks and multi-block verify (gfx950).
//
// Replaces, per attention layer, the reference's static-cache forward
// (speculative_decoding/adapters/base.py:161-265 with SDAR's qkv,
// sdar/modeling_sdar.py:250-262):
//   q = q_norm(q_proj(x)); k = k_norm(k_proj(x)); v = v_proj(x)
//   q, k = apply_rotary_pos_emb(q, k, cos, sin)
//   key_cache.index_copy_(2, slots, k) ... (per GQA replica)      -> qkv_rope_cache_kernel
//   out = F.scaled_dot_product_attention(q, K, V, attn_mask=bool)  -> attn_partial + attn_combine
//
// Cache layout, per layer (one sequence) and KV head, L a multiple of 32: K and
// V in tiles laid out in the order the MFMA operands are read, so that every
// wave-wide 16-byte load covers 1 KB of contiguous memory (8 whole cache
// lines, where a row-major [L, D] or [D, L] layout touches 16 lines per load):
//   K: [L/16][16 dim chunks of 8][16 keys][8 dims]
//      (slot s, dim d) -> ((s/16 * 16 + d/8) * 16 + s%16) * 8 + d%8
//   V: [L/32][8 dim tiles of 16][16 dims][4 key quads][2 halves][4 keys]
//      (slot s, dim d) -> ((((s/32 * 8 + d/16) * 16 + d%16) * 4 + s/4%4) * 2 + s/16%2) * 4 + s%4
// The KV heads are not replicated per query head (the reference's "expand"
// mode copies each of them n_rep times); every query head reads its group's
// KV head, so the cache and its traffic are n_rep times smaller.  The products:
//   S^T = K . Q^T   A = K tile (16 keys x 32 dims), B = Q^T (32 dims x 16 rows)
//   O^T = Vt . P^T  A = Vt tile (16 dims x 32 keys), B = P^T (32 keys x 16 rows)
// and P^T never leaves registers: the S^T result lane (g, r) holds keys
// 4g..4g+3 of each 16-key tile for row r, which, with the MFMA's k-slots
// assigned as {tile 0: 4g..4g+3, tile 1: 4g..4g+3}, is exactly that lane's B
// operand of the second product (A and B only need to agree on the k order).
// Query rows are the (query head, token) pairs of one KV head's group,
// row = i * M + m for query head h * n_rep + i, padded to 16-row blocks.
//
// Short contexts: one workgroup per KV head, its waves taking the 32-key steps
// in turn and merging their online-softmax states in LDS (one launch).  Long
// contexts: the key range is split into chunks, one workgroup per (chunk, KV
// head); each keeps an online softmax (running max and sum per row) and writes
// its unnormalised partial output; attn_combine merges the chunks in chunk
// order.  Both orders are fixed: bit-reproducible.
#include <algorithm>
#include <type_traits>

#include "simsd_common.hpp"
#include "simsd_kernels.h"

namespace simsd {
namespace {

constexpr int kHeadDim = 128;
constexpr int kDSteps = kHeadDim / 32;      // MFMA k-steps over the head dim
constexpr int kDTiles = kHeadDim / 16;      // 16-dim tiles of the output
constexpr int kKeyStep = 32;                // keys per inner step (two 16-key tiles)

// ---------------------------------------------------------- lane exchanges
// Combine over the four 16-lane groups (lane bits 4 and 5): the gfx950 swaps
// applied to (v, v) hand every lane the values of its row pair and then of
// its half-wave pair, combined lower-first, so all lanes end equal.
template <typename Combine>
SIMSD_DEV float across_groups(float v, Combine combine) {
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = combine(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return combine(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

template <int DT> SIMSD_DEV uint32_t pack2(float lo, float hi);
template <> SIMSD_DEV uint32_t pack2<kBF16>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
template <> SIMSD_DEV uint32_t pack2<kF16>(float lo, float hi) {
  return f32_to_h16<kF16>(lo) | (f32_to_h16<kF16>(hi) << 16);
}

// ------------------------------------------------ q/k norm, RoPE, cache write
// Element index of (slot s, dim d) in one KV head's K and V tiles.
SIMSD_DEV int64_t k_tile_index(int64_t s, int d) {
  return (((s >> 4) * 16 + (d >> 3)) * 16 + (s & 15)) * 8 + (d & 7);
}
SIMSD_DEV int64_t v_tile_index(int64_t s, int d) {
  return (((((s >> 5) * 8 + (d >> 4)) * 16 + (d & 15)) * 4 + ((s >> 2) & 3)) * 2 + ((s >> 4) & 1)) * 4 + (s & 3);
}

struct QkvArgs {
  const char* qkv;            // [M, (Hq + 2 Hkv) * D]: q heads, then k heads, then v heads
  int64_t sqkv;               // row stride (elements)
  const char* qn;             // q_norm weight [D] or null
  const char* kn;             // k_norm weight [D] or null
  float eps;
  const char* cos;            // [n_pos, D] rows (stride scs)
  const char* sin;
  int64_t scs, n_pos;
  const int64_t* pos;         // [M]
  const int64_t* slots;       // [M] cache slots written
  const int64_t* slots2;      // [M] second slots (permanent copies) or null
  char* kc;                   // K tiles, head stride sh (elements)
  char* vc;                   // V tiles, head stride sh
  int64_t sh;
  int64_t L;
  char* qo;                   // [M, Hq, D]
  int64_t sqo_m, sqo_h;
  int Hq, Hkv;
  // in place of qkv: the projection's fp32 split-K partials [split][M][N],
  // N = (Hq + 2 Hkv) * D, summed here in split order and rounded to the dtype
  const float* part;
  int split;
  int64_t part_mn;
};

constexpr int kQkvMaxSplit = 8;   // partials the cache-write launch sums

// grid (M, head groups of 8): one wave per (token, head); lane l owns dims l
// and l + 64, the two halves rotate_half pairs.  All of a wave's loads are
// issued before its arithmetic.  Rounding points of the bf16 reference: the
// norm is the stock RMSNorm (weight * dtype(x * r), r in fp32), then
// q_embed = dtype(dtype(q * cos) + dtype(rotate_half(q) * sin)).
// The fields the first loads depend on come as leading scalar arguments,
// which the build preloads into SGPRs; the rest of QkvArgs is read after.
template <int DT, bool PART>
__global__ __launch_bounds__(512) void qkv_rope_cache_kernel(const char* __restrict__ qkv, const int64_t* __restrict__ pos,
                                                             const int64_t* __restrict__ slots, const char* qn,
                                                             const char* kn, int sqkv, int Hq, int Hkv, QkvArgs a) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  const int lane = threadIdx.x & 63;
  const int hh = (int)blockIdx.y * (int)(blockDim.x >> 6) + (int)(threadIdx.x >> 6);
  if (hh >= Hq + 2 * Hkv) return;
  const int64_t m = blockIdx.x;
  const int64_t p = pos[m];
  const int64_t s1 = slots[m];
  const int64_t s2 = a.slots2 != nullptr ? a.slots2[m] : -1;
  const bool pos_ok = p >= 0 && p < a.n_pos;
  const bool s1_ok = s1 >= 0 && s1 < a.L;
  const bool s2_ok = s2 >= 0 && s2 < a.L;
  const int d0 = lane, d1 = lane + 64;
  const bool is_v = hh >= Hq + Hkv;
  const bool is_q = hh < Hq;
  const char* nwt = is_q ? qn : kn;
  float x0, x1;
  if constexpr (PART) {
    // the partials of this row and head, all loaded before any is summed
    // (past the split count the loads re-read partial 0 and are dropped); the
    // sum starts from 0 above one partial, as thin_reduce_kernel's does, so
    // the rounded values equal the reduced projection's
    const float* pr = a.part + m * sqkv + (int64_t)hh * kHeadDim;
    float p0[kQkvMaxSplit], p1[kQkvMaxSplit];
#pragma unroll
    for (int s = 0; s < kQkvMaxSplit; ++s) {
      const float* ps = pr + (s < a.split ? s : 0) * a.part_mn;
      p0[s] = ps[d0];
      p1[s] = ps[d1];
    }
    float v0 = a.split > 1 ? 0.f + p0[0] : p0[0], v1 = a.split > 1 ? 0.f + p1[0] : p1[0];
#pragma unroll
    for (int s = 1; s < kQkvMaxSplit; ++s) {
      v0 = s < a.split ? v0 + p0[s] : v0;
      v1 = s < a.split ? v1 + p1[s] : v1;
    }
    x0 = round_to<DT>(v0);
    x1 = round_to<DT>(v1);
  } else {
    const char* src = qkv + (m * sqkv + (int64_t)hh * kHeadDim) * ES;
    x0 = load_elem<DT>(src, d0);
    x1 = load_elem<DT>(src, d1);
  }
  float w0 = 1.f, w1 = 1.f, c0 = 0.f, c1 = 0.f, n0 = 0.f, n1 = 0.f;
  if (!is_v) {
    if (nwt != nullptr) {
      w0 = load_elem<DT>(nwt, d0);
      w1 = load_elem<DT>(nwt, d1);
    }
    if (pos_ok) {
      const char* cr = a.cos + p * a.scs * ES;
      const char* sr = a.sin + p * a.scs * ES;
      c0 = load_elem<DT>(cr, d0); c1 = load_elem<DT>(cr, d1);
      n0 = load_elem<DT>(sr, d0); n1 = load_elem<DT>(sr, d1);
    }
  }
  if (is_v) {   // v head: copy into the V tiles
    char* base = a.vc + (int64_t)(hh - Hq - Hkv) * a.sh * ES;
    if (s1_ok) {
      store_elem<DT>(base, v_tile_index(s1, d0), x0);
      store_elem<DT>(base, v_tile_index(s1, d1), x1);
    }
    if (s2_ok) {
      store_elem<DT>(base, v_tile_index(s2, d0), x0);
      store_elem<DT>(base, v_tile_index(s2, d1), x1);
    }
    return;
  }
  if (nwt != nullptr) {
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = 1.f / sqrtf(ss / (float)kHeadDim + a.eps);
    x0 = round_to<DT>(w0 * round_to<DT>(x0 * r));
    x1 = round_to<DT>(w1 * round_to<DT>(x1 * r));
  }
  float y0 = 0.f, y1 = 0.f;
  if (pos_ok) {
    y0 = round_to<DT>(round_to<DT>(x0 * c0) + round_to<DT>(-x1 * n0));
    y1 = round_to<DT>(round_to<DT>(x1 * c1) + round_to<DT>(x0 * n1));
  }
  if (is_q) {
    char* dst = a.qo + (m * a.sqo_m + (int64_t)hh * a.sqo_h) * ES;
    store_elem<DT>(dst, d0, y0);
    store_elem<DT>(dst, d1, y1);
  } else if (pos_ok) {
    char* base = a.kc + (int64_t)(hh - Hq) * a.sh * ES;
    if (s1_ok) {
      store_elem<DT>(base, k_tile_index(s1, d0), y0);
      store_elem<DT>(base, k_tile_index(s1, d1), y1);
    }
    if (s2_ok) {
      store_elem<DT>(base, k_tile_index(s2, d0), y0);
      store_elem<DT>(base, k_tile_index(s2, d1), y1);
    }
  }
}

// ------------------------------------------------------------ attention
struct AttnArgs {
  const char* q;              // [M, Hq, D]
  int64_t sq_m, sq_h;
  const char* kc;             // K tiles, head stride sh (elements)
  const char* vc;             // V tiles, head stride sh
  int64_t sh, L_cap;
  const uint8_t* mask;        // [M, >= L_valid] (nonzero = visible) or null
  int64_t smask;
  int64_t M;
  int n_rep, Hkv;
  int64_t L_valid, chunk, wave_chunk;
  int n_chunks;
  float scale;
  int rows, rows_pad;         // n_rep * M, padded to 16
  const int64_t* lv_dev;      // device-side valid slot count (<= L_valid) or null
  float* o_part;              // [Hkv][n_chunks][rows_pad][D]
  float2* ml_part;            // [Hkv][n_chunks][rows_pad]
  unsigned* arrivals;         // [Hkv] workgroups of the split head form done (0 between calls)
};

// Loads are unconditional -- the caller points an unused lane at a valid
// address -- and unused values are replaced afterwards: a load under a branch
// would make the compiler wait for it at the join, serialising the batch.
SIMSD_DEV u32x4_t load16_sel(const char* p, bool ok) {
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
  return ok ? v : zero4();
}


constexpr float kLog2e = 1.4426950408889634f;

// A wave's view of one KV head: descriptors over the head's K and V tiles and
// per-lane byte offsets, so each 32-key step's loads are one add each.  A
// step at slot c (a multiple of 32) starts at byte c * 256 of both tile
// arrays; within it, lane (g, r) reads
//   K tile t, dim step ds: 16 bytes at t*4096 + (4*ds + g)*256 + r*16
//     (keys c + 16t + r, dims 32*ds + 8g .. +8: the A operand of S^T)
//   V dim tile dt:         16 bytes at dt*1024 + r*64 + g*16
//     (dim 16*dt + r, keys c + 4g .. +4 then c + 16 + 4g .. +4: the A operand
//      of O^T with the k-slots of P^T)
// so every load instruction covers 1 KB of contiguous memory.  Slots past the
// valid range read stale cache values: their scores are replaced by -inf
// (p = 0) and their V by zeros (attn_step); past L_cap they read as zero.
// mask: all M rows.
template <int RBW>
struct WaveKV {
  rsrc_t rk, rv, rm;
  uint32_t k_off, v_off, m_off[RBW];
  int c_oob;   // a step slot whose K and V bytes all lie past the descriptors' range
};

template <int DT, int RBW>
SIMSD_DEV WaveKV<RBW> wave_kv(const char* kc, const char* vc, int64_t sh, uint32_t head_bytes, const AttnArgs& a, int h,
                              const int (&tok)[RBW], int g, int r) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  WaveKV<RBW> w;
  w.rk = make_rsrc(kc + (int64_t)h * sh * ES, head_bytes);
  w.rv = make_rsrc(vc + (int64_t)h * sh * ES, head_bytes);
  w.rm = make_rsrc(a.mask, a.mask != nullptr ? (uint32_t)(a.M * a.smask) : 0u);
  w.k_off = (uint32_t)(g * 256 + r * 16);
  w.v_off = (uint32_t)(r * 64 + g * 16);
  w.c_oob = (int)(head_bytes / 256u);
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) w.m_off[rb] = (uint32_t)(tok[rb] * a.smask + 4 * g);
  return w;
}
template <int DT, int RBW>
SIMSD_DEV WaveKV<RBW> wave_kv(const AttnArgs& a, int h, const int (&tok)[RBW], int g, int r) {
  return wave_kv<DT, RBW>(a.kc, a.vc, a.sh, (uint32_t)(a.L_cap * kHeadDim * DTypeInfo<DT>::kSize), a, h, tok, g, r);
}

// Operands of one 32-key step: K tiles (A of S^T = K.Q^T), V tiles (A of
// O^T = Vt.P^T) and, per row block, the 2 x 4 mask bytes of the lane's keys.
template <int RBW>
struct StepBuf {
  u32x4_t kf[2][kDSteps];
  u32x4_t vf[kDTiles];
  uint32_t mk[RBW][2];
};

// The step to prefetch after the one at c: c_next while it starts before
// c_end, else a slot past the K/V range, whose loads the buffer range check
// answers with zeros without a memory request (the step is never computed;
// a cache larger than the valid length would otherwise stream 16 KB of
// stale slots per wave at the end of its range).  Uniform across the wave.
template <int RBW>
SIMSD_DEV int next_step(const WaveKV<RBW>& w, int c_next, int c_end) {
  return c_next < c_end ? c_next : w.c_oob;
}

template <int DT, int RBW>
SIMSD_DEV void attn_load(const AttnArgs& a, const WaveKV<RBW>& w, int c, StepBuf<RBW>& b) {
  static_assert(DTypeInfo<DT>::kSize == 2, "16-bit K/V");
  const uint32_t base = (uint32_t)c * 256u;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int ds = 0; ds < kDSteps; ++ds)
      b.kf[t][ds] = buf_load16<kAuxKeep>(w.rk, base + w.k_off + (uint32_t)(t * 4096 + ds * 1024));
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt) b.vf[dt] = buf_load16<kAuxKeep>(w.rv, base + w.v_off + (uint32_t)(dt * 1024));
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb)
#pragma unroll
    for (int t = 0; t < 2; ++t) b.mk[rb][t] = a.mask != nullptr ? buf_load4(w.rm, w.m_off[rb] + c + 16 * t) : ~0u;
}

// One 32-key step of the online softmax for RBW row blocks: S^T = K.Q^T,
// mask, running max / sum per row in the log2 domain (scores scaled by
// scale * log2(e), p = 2^(s - m)), O^T += Vt.P^T.  The accumulators are
// rescaled only when some row's maximum moved.
template <int DT, int RBW>
SIMSD_DEV void attn_step(const AttnArgs& a, const u32x4_t (&qf)[RBW][kDSteps], const bool (&row_ok)[RBW],
                         const StepBuf<RBW>& b, int c, int c_end, int g, float (&m_run)[RBW],
                         float (&l_run)[RBW], f32x4_t (&acc)[RBW][kDTiles]) {
  const float sl2 = a.scale * kLog2e;
  // V of keys past the valid length is zeroed in the step that straddles it:
  // those slots hold whatever an earlier forward left, and an Inf there would
  // turn p = 0 into 0 * Inf = NaN in the product.  Lane (g, r) holds keys
  // c + 4g + {0..3} (dwords 0, 1) and c + 16 + 4g + {0..3} (dwords 2, 3),
  // two per dword, the lower key in the low half.  c and c_end are uniform
  // across the wave, so the branch is too.
  u32x4_t vf[kDTiles];
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt) vf[dt] = b.vf[dt];
  if (c + 32 > c_end) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k0 = c + 4 * g + (j >> 1) * 16 + (j & 1) * 2;
      const uint32_t keep = (k0 < c_end ? 0x0000ffffu : 0u) | (k0 + 1 < c_end ? 0xffff0000u : 0u);
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) vf[dt][j] &= keep;
    }
  }
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    f32x4_t s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < kDSteps; ++ds) s[t] = Mfma<DT>::step(b.kf[t][ds], qf[rb][ds], s[t]);
    }
    // lane (g, r): s[t][j] = S^T[key c + 16t + 4g + j][row rb*16 + r]
    float sv[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool vis = row_ok[rb] && c + 16 * t + 4 * g + j < c_end && ((b.mk[rb][t] >> (8 * j)) & 0xffu) != 0;
        sv[t][j] = vis ? s[t][j] * sl2 : -INFINITY;
        mx = fmaxf(mx, sv[t][j]);
      }
    mx = across_groups(mx, [](float x, float y) { return fmaxf(x, y); });
    const float m_new = fmaxf(m_run[rb], mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;   // no visible key yet: every p is 0
    const float alpha = __builtin_amdgcn_exp2f(m_run[rb] - m_use);
    float p[2][4];
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[t][j] = __builtin_amdgcn_exp2f(sv[t][j] - m_use);
        ps += p[t][j];
      }
    ps = across_groups(ps, [](float x, float y) { return x + y; });
    l_run[rb] = l_run[rb] * alpha + ps;
    const bool moved = m_run[rb] != -INFINITY && m_new != m_run[rb];
    m_run[rb] = m_new;
    if (__any(moved)) {
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) acc[rb][dt] *= alpha;
    }
    const u32x4_t pf = u32x4_t{pack2<DT>(p[0][0], p[0][1]), pack2<DT>(p[0][2], p[0][3]),
                               pack2<DT>(p[1][0], p[1][1]), pack2<DT>(p[1][2], p[1][3])};
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) acc[rb][dt] = Mfma<DT>::step(vf[dt], pf, acc[rb][dt]);
  }
}

// grid (n_chunks, Hkv, row groups), 4 waves (KSPLIT) or W waves.
//   KSPLIT: every wave holds all RBW row blocks and a quarter of the
//     workgroup's key chunk; the four online-softmax states merge through LDS.
//   otherwise: the waves share the key chunk and own row blocks
//     [(z*W + w)*RBW, (z*W + w + 1)*RBW) of row group z.
// Each wave runs its 32-key steps with the next step's K/Vt loads in flight.
template <int DT, int RBW, bool KSPLIT>
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs a) {
  constexpr int ES = DTypeInfo<DT>::kSize;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int chunk_id = blockIdx.x;
  const int h = blockIdx.y;
  const int rb0 = KSPLIT ? 0 : ((int)blockIdx.z * nw + wv) * RBW;
  if (!KSPLIT && rb0 * 16 >= a.rows) return;   // no rows for this wave (whole wave exits)

  // Q^T fragments (B operand): row = rb*16 + r, dims ds*32 + 8g .. +8
  u32x4_t qf[RBW][kDSteps];
  int tok[RBW];
  bool row_ok[RBW];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    const int row = (rb0 + rb) * 16 + r;
    row_ok[rb] = row < a.rows;
    const int i = row_ok[rb] ? row / (int)a.M : 0;
    tok[rb] = row_ok[rb] ? row % (int)a.M : 0;
    const int hq = h * a.n_rep + i;
    const char* qp = a.q + ((int64_t)tok[rb] * a.sq_m + (int64_t)hq * a.sq_h) * ES;
#pragma unroll
    for (int ds = 0; ds < kDSteps; ++ds) qf[rb][ds] = load16_sel(qp + (ds * 32 + 8 * g) * ES, row_ok[rb]);
  }

  float m_run[RBW], l_run[RBW];
  f32x4_t acc[RBW][kDTiles];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) acc[rb][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  int64_t lv = a.L_valid;
  if (a.lv_dev != nullptr) {
    const int64_t d = *a.lv_dev;
    lv = d < 0 ? 0 : (d < lv ? d : lv);
  }
  const int64_t chunk_lo = (int64_t)chunk_id * a.chunk;
  if (chunk_lo >= lv) return;   // past the valid length: the merge skips this chunk
  const int64_t chunk_hi = min(lv, chunk_lo + a.chunk);
  const int64_t c_begin = KSPLIT ? min(chunk_hi, chunk_lo + (int64_t)wv * a.wave_chunk) : chunk_lo;
  const int64_t c_end = KSPLIT ? min(chunk_hi, c_begin + a.wave_chunk) : chunk_hi;
  // the next step's loads are issued before this step's arithmetic; past
  // c_end they read zeros or stale slots, whose p is 0 and V zeroed
  StepBuf<RBW> bA, bB;
  if (c_begin < c_end) {
    const WaveKV<RBW> w = wave_kv<DT, RBW>(a, h, tok, g, r);
    const int ce = (int)c_end;
    attn_load<DT, RBW>(a, w, (int)c_begin, bA);
    for (int c = (int)c_begin;; c += 2 * kKeyStep) {
      attn_load<DT, RBW>(a, w, next_step(w, c + kKeyStep, ce), bB);
      attn_step<DT, RBW>(a, qf, row_ok, bA, c, ce, g, m_run, l_run, acc);
      if (c + kKeyStep >= ce) break;
      attn_load<DT, RBW>(a, w, next_step(w, c + 2 * kKeyStep, ce), bA);
      attn_step<DT, RBW>(a, qf, row_ok, bB, c + kKeyStep, ce, g, m_run, l_run, acc);
      if (c + 2 * kKeyStep >= ce) break;
    }
  }

  const int64_t base_row = ((int64_t)h * a.n_chunks + chunk_id) * a.rows_pad;
  if constexpr (KSPLIT) {
    // merge the four waves' states in wave order: LDS o[w][row][d], ml[w][row]
    __shared__ __attribute__((aligned(16))) float o_sh[4][RBW * 16][kHeadDim];
    __shared__ float2 ml_sh[4][RBW * 16];
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
      const int row = rb * 16 + r;
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt)
        *reinterpret_cast<f32x4_t*>(&o_sh[wv][row][dt * 16 + 4 * g]) = acc[rb][dt];
      if (g == 0) ml_sh[wv][row] = make_float2(m_run[rb], l_run[rb]);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < RBW * 16 * kHeadDim; e += blockDim.x) {
      const int row = e / kHeadDim, d = e % kHeadDim;
      if (row >= a.rows) continue;
      float mx = -INFINITY;
      for (int w = 0; w < nw; ++w) mx = fmaxf(mx, ml_sh[w][row].x);
      float o = 0.f, l = 0.f;
      for (int w = 0; w < nw; ++w) {
        const float2 ml = ml_sh[w][row];
        const float wt = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
        o += o_sh[w][row][d] * wt;
        l += ml.y * wt;
      }
      a.o_part[(base_row + row) * kHeadDim + d] = o;
      if (d == 0) a.ml_part[base_row + row] = make_float2(mx, l);
    }
  } else {
    // lane (g, r): acc[rb][dt][j] = O^T[dim dt*16 + 4g + j][row rb*16 + r]
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
      const int row = (rb0 + rb) * 16 + r;
      if (!row_ok[rb]) continue;
      float* op = a.o_part + (base_row + row) * kHeadDim;
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt)
        *reinterpret_cast<f32x4_t*>(op + dt * 16 + 4 * g) = acc[rb][dt];
      if (g == 0) a.ml_part[base_row + row] = make_float2(m_run[rb], l_run[rb]);
    }
  }
}

// Up to 32 query rows per KV head over a short context: grid (S_max, Hkv),
// W waves per workgroup.  From the valid length the kernel takes S <= S_max
// workgroups per KV head (one up to kSplitMin slots, else one 32-key step per
// wave) and deals the steps out in turn (step i to workgroup (i / W) % S,
// wave i % W), so a wave's first step does not depend on the valid length and
// its loads are issued before that length is read; the next step's loads stay
// in flight during each step.  The W online-softmax states merge in LDS
// (fixed wave order).  S = 1: the normalised rows go straight to the output.
// S > 1: each workgroup writes its unnormalised rows and (max, sum) to the
// workspace, and the last to arrive (an arrival counter per KV head, reset to
// 0 by that workgroup) merges the S partials in workgroup order.  One launch
// either way.  W = 4 for one 16-row block and for two (kHeadW1, kHeadW2).
#ifndef SIMSD_HEAD_MAX_SLOTS
#define SIMSD_HEAD_MAX_SLOTS 4096   // measured: the split head form beats the chunked one up to here
#endif
constexpr int kHeadMaxSlots = SIMSD_HEAD_MAX_SLOTS;
// valid lengths up to which one workgroup per KV head takes all the steps
// (16 and 32 rows): below them the hand-over costs more than the split saves
// (16 rows, measured with the merge reading only the valid rows of exactly S
// partials: 400 slots 10.15 -> 8.74 us split, 200 slots 8.09 one workgroup
// against 8.41 split)
#ifndef SIMSD_HEAD_SPLIT_MIN_SLOTS1
#define SIMSD_HEAD_SPLIT_MIN_SLOTS1 256
#endif
#ifndef SIMSD_HEAD_SPLIT_MIN_SLOTS2
#define SIMSD_HEAD_SPLIT_MIN_SLOTS2 384
#endif
constexpr int kHeadSplitMinSlots1 = SIMSD_HEAD_SPLIT_MIN_SLOTS1;
constexpr int kHeadSplitMinSlots2 = SIMSD_HEAD_SPLIT_MIN_SLOTS2;
// Hand-over of the partials between the workgroups of a KV head (which may
// sit on different XCDs, each with its own L2):
//   2  formal: every shared value is a relaxed atomic written through to
//      memory and read past every cache level, and the arrival counter is a
//      release fetch_add whose last arriver acquires, so the language's memory
//      model orders the partials before their reads;
//   1  the same stores and loads, ordered by the stores' completion
//      (s_waitcnt) before a relaxed arrival;
//   0  plain stores and loads with device-scope fences.
#ifndef SIMSD_HEAD_SPLIT_SYNC
#define SIMSD_HEAD_SPLIT_SYNC 2
#endif
SIMSD_DEV void put_through(float* p, float v) {
  if (SIMSD_HEAD_SPLIT_SYNC) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  else *p = v;
}
SIMSD_DEV void put_through2(float* p, float v0, float v1) {   // p 8-byte aligned
  const uint64_t b = (uint64_t)__float_as_uint(v0) | ((uint64_t)__float_as_uint(v1) << 32);
  if (SIMSD_HEAD_SPLIT_SYNC) __hip_atomic_store(reinterpret_cast<uint64_t*>(p), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  else *reinterpret_cast<uint64_t*>(p) = b;
}
SIMSD_DEV float get_through(const float* p) {
  if (SIMSD_HEAD_SPLIT_SYNC) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  return *p;
}
// Count this workgroup's arrival at KV head h; true in the last to arrive.
SIMSD_DEV bool arrive_last(unsigned* counter, unsigned n) {
  if (SIMSD_HEAD_SPLIT_SYNC == 2)
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
  if (SIMSD_HEAD_SPLIT_SYNC == 1) {
    __builtin_amdgcn_s_waitcnt(0);   // the partial is in memory before the arrival is counted
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
  }
  __threadfence();
  const bool last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
  __threadfence();
  return last;
}
#ifndef SIMSD_HEAD_MAX_SPLIT
#define SIMSD_HEAD_MAX_SPLIT 8
#endif
constexpr int kHeadMaxSplit = SIMSD_HEAD_MAX_SPLIT;   // workgroups per KV head in the split head form
// waves per workgroup of the head form: one 16-row block, two (measured
// with the 16-byte hand-over: 4 waves for one block beat 8 from 128 to 2048
// slots, 8 rows at 1024 slots 10.6 -> 9.3 us)
#ifndef SIMSD_HEAD_W1
#define SIMSD_HEAD_W1 4
#endif
constexpr int kHeadW1 = SIMSD_HEAD_W1;
constexpr int kHeadW2 = 4;

// LDS of the head form: the waves' states, the merge weights and the split
// hand-over's flag.
template <int RBW, int W, int MAXS = kHeadMaxSplit>
struct HeadShared {
  static constexpr int ROWS = RBW * 16;
  static constexpr int OSTR = kHeadDim + 4;   // padded rows: the b128 writes of 16 rows spread over the banks
  float o[W][ROWS][OSTR];
  float2 ml[W][ROWS];
  float wt[W][ROWS];
  float l[ROWS];
  float mx[ROWS];
  float wts[MAXS][ROWS];
  int last;
};

// Workgroups a KV head's `steps` 32-key steps are dealt to (the caller caps
// it by the grid): one step a wave up to SIMSD_HEAD_SPW_SWITCH steps, then
// SIMSD_HEAD_SPW_X2 / 2 steps a wave -- past ~900 slots a partial fewer to
// merge costs less than a wave's second step.  The host sizes the grid with
// the same rule from its bound on the valid length.
#ifndef SIMSD_HEAD_SPW_X2
#define SIMSD_HEAD_SPW_X2 3
#endif
#ifndef SIMSD_HEAD_SPW_SWITCH
#define SIMSD_HEAD_SPW_SWITCH 28
#endif
__host__ __device__ inline int head_split(int steps, int W) {
  if (steps <= SIMSD_HEAD_SPW_SWITCH) return (steps + W - 1) / W;
  const int per = W * SIMSD_HEAD_SPW_X2;   // twice the steps a workgroup takes
  return (2 * steps + per - 1) / per;
}

// The last arriver's merge of the NS partials of KV head h, in workgroup
// order.  The partial rows and the (max, sum) pairs are all loaded before any
// is used, so the merge waits for one round trip: plain 16-byte loads, ordered
// after the writers' stores by the arrival's release and the last arriver's
// acquire (which also drops this CU's stale cache lines).  A pass whose units
// all lie in the padding rows (rows <= 8 of a 16-row block: the draft's 4
// tokens x 2 query heads) loads nothing (a workgroup-uniform test); rows past
// rows in a pass that does load read the workspace's row padding and are
// dropped.
template <int DT, int RBW, int W, int MAXS, int NS>
SIMSD_DEV void head_merge(HeadShared<RBW, W, MAXS>& sh, const AttnArgs& a, int h, int rows, int M, int n_rep,
                          char* __restrict__ out, int64_t so_m, int64_t so_h) {
  static_assert(NS >= 1 && NS <= MAXS, "partials the shared arrays hold");
  constexpr int ROWS = RBW * 16;
  constexpr int kPer4 = ROWS * kHeadDim / 4 / (64 * W);
  static_assert(kPer4 >= 1 && ROWS * kHeadDim % (4 * 64 * W) == 0, "whole float4 units per thread");
  const float4* pO = reinterpret_cast<const float4*>(a.o_part + (int64_t)h * NS * ROWS * kHeadDim);
  const float2* pML = a.ml_part + (int64_t)h * NS * ROWS;
  float4 v4[kPer4][NS];
  const int units = rows * (kHeadDim / 4);
#pragma unroll
  for (int i = 0; i < kPer4; ++i) {
    const int e = (int)threadIdx.x + i * 64 * W;   // float4 unit: row e / 32, dims 4 (e % 32) ..
    if (i == 0 || i * 64 * W < units) {
#pragma unroll
      for (int q = 0; q < NS; ++q)
        v4[i][q] = pO[(q * ROWS + e / (kHeadDim / 4)) * (kHeadDim / 4) + e % (kHeadDim / 4)];
    }
  }
  if (threadIdx.x < rows) {
    const int row = threadIdx.x;
    float pm[NS], pl[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const float2 ml = pML[q * ROWS + row];
      pm[q] = ml.x;
      pl[q] = ml.y;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < NS; ++q) mx = fmaxf(mx, pm[q]);
    float l = 0.f;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const float wt = pm[q] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(pm[q] - mx);
      sh.wts[q][row] = wt;
      l += pl[q] * wt;
    }
    sh.l[row] = l;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPer4; ++i) {
    const int e = (int)threadIdx.x + i * 64 * W;
    const int row = e / (kHeadDim / 4), d = (e % (kHeadDim / 4)) * 4;
    if (row < rows) {
      float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        const float wt = sh.wts[q][row];
        o0 += v4[i][q].x * wt;
        o1 += v4[i][q].y * wt;
        o2 += v4[i][q].z * wt;
        o3 += v4[i][q].w * wt;
      }
      const float l = sh.l[row];
      const int ih = row / M;
      const int64_t m = row % M;
      char* orow = out + (m * so_m + (int64_t)(h * n_rep + ih) * so_h + d) * DTypeInfo<DT>::kSize;
      store_elem<DT>(orow, 0, l > 0.f ? o0 / l : 0.f);
      store_elem<DT>(orow, 1, l > 0.f ? o1 / l : 0.f);
      store_elem<DT>(orow, 2, l > 0.f ? o2 / l : 0.f);
      store_elem<DT>(orow, 3, l > 0.f ? o3 / l : 0.f);
    }
  }
}

// head_merge for NS = S, 2 <= S <= MAXS (S is uniform across the workgroup).
template <int DT, int RBW, int W, int MAXS, int NS = 2>
SIMSD_DEV void head_merge_n(int S, HeadShared<RBW, W, MAXS>& sh, const AttnArgs& a, int h, int rows, int M,
                            int n_rep, char* __restrict__ out, int64_t so_m, int64_t so_h) {
  if constexpr (NS >= MAXS) {
    head_merge<DT, RBW, W, MAXS, MAXS>(sh, a, h, rows, M, n_rep, out, so_m, so_h);
  } else {
    if (S == NS) head_merge<DT, RBW, W, MAXS, NS>(sh, a, h, rows, M, n_rep, out, so_m, so_h);
    else head_merge_n<DT, RBW, W, MAXS, NS + 1>(S, sh, a, h, rows, M, n_rep, out, so_m, so_h);
  }
}

// The head form's tail, shared by both head kernels: the W waves' online
// softmax states merge in LDS (fixed wave order); S = 1 writes the
// normalised rows; S > 1 writes this workgroup's partial, counts its arrival
// and the last to arrive merges the S partials in workgroup order.
template <int DT, int RBW, int W, int MAXS = kHeadMaxSplit>
SIMSD_DEV void head_finish(HeadShared<RBW, W, MAXS>& sh, const f32x4_t (&acc)[RBW][kDTiles], const float (&m_run)[RBW],
                           const float (&l_run)[RBW], const AttnArgs& a, int sp, int S, int h, int rows, int M,
                           int n_rep, char* __restrict__ out, int64_t so_m, int64_t so_h) {
  constexpr int ROWS = RBW * 16;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  // lane (g, r): acc[rb][dt][j] = O^T[dim dt*16 + 4g + j][row rb*16 + r]
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt)
      *reinterpret_cast<f32x4_t*>(&sh.o[wv][rb * 16 + r][dt * 16 + 4 * g]) = acc[rb][dt];
    if (g == 0) sh.ml[wv][rb * 16 + r] = make_float2(m_run[rb], l_run[rb]);
  }
  __syncthreads();
  if (threadIdx.x < ROWS) {
    const int row = threadIdx.x;
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < W; ++v) mx = fmaxf(mx, sh.ml[v][row].x);
    float l = 0.f;
#pragma unroll
    for (int v = 0; v < W; ++v) {
      const float2 ml = sh.ml[v][row];
      const float wt = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
      sh.wt[v][row] = wt;
      l += ml.y * wt;
    }
    sh.l[row] = l;
    sh.mx[row] = mx;
  }
  __syncthreads();
  auto put = [&](int row, int d, float o, float l) {
    const int i = row / M;
    const int64_t m = row % M;
    store_elem<DT>(out, m * so_m + (int64_t)(h * n_rep + i) * so_h + d, l > 0.f ? o / l : 0.f);
  };
  if (S == 1) {
    for (int e = threadIdx.x; e < ROWS * kHeadDim; e += 64 * W) {
      const int row = e / kHeadDim, d = e % kHeadDim;
      if (row >= rows) break;
      float o = 0.f;
#pragma unroll
      for (int v = 0; v < W; ++v) o += sh.o[v][row][d] * sh.wt[v][row];
      put(row, d, o, sh.l[row]);
    }
    return;
  }
  // this workgroup's partial: [h][sp][row][d] and (max, sum) [h][sp][row],
  // two values per write-through store
  const int64_t pbase = ((int64_t)h * S + sp) * ROWS;
  for (int e = threadIdx.x; e < ROWS * kHeadDim / 2; e += 64 * W) {
    const int row = e / (kHeadDim / 2), d = (e % (kHeadDim / 2)) * 2;
    if (row >= rows) break;
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int v = 0; v < W; ++v) {
      o0 += sh.o[v][row][d] * sh.wt[v][row];
      o1 += sh.o[v][row][d + 1] * sh.wt[v][row];
    }
    put_through2(a.o_part + (pbase + row) * kHeadDim + d, o0, o1);
  }
  if (threadIdx.x < rows)
    put_through2(reinterpret_cast<float*>(a.ml_part + pbase + threadIdx.x), sh.mx[threadIdx.x], sh.l[threadIdx.x]);
  // Every thread's stores precede the barrier; thread 0's arrival follows it
  // (the workgroup barrier orders them at workgroup scope, the arrival's
  // release extends that to the agent).
  __syncthreads();
  if (threadIdx.x == 0) sh.last = arrive_last(a.arrivals + h, (unsigned)S);
  __syncthreads();
  if (!sh.last) return;
  // the merge, instantiated for the exact partial count (a chain of uniform
  // tests on S), so no load re-reads a partial past S
  head_merge_n<DT, RBW, W, MAXS>(S, sh, a, h, rows, M, n_rep, out, so_m, so_h);
  if (threadIdx.x == 0) __hip_atomic_store(a.arrivals + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The fields the first loads depend on come as leading scalar arguments,
// which the build preloads into SGPRs; the rest of AttnArgs is read after.
template <int DT, int RBW, int W>
__global__ __launch_bounds__(64 * W) void attn_head_kernel(const char* __restrict__ q, const char* __restrict__ kc,
                                                           const char* __restrict__ vc,
                                                           const int64_t* __restrict__ lv_dev, int sq_m, int sq_h,
                                                           int sh, uint32_t head_bytes, int M, int n_rep, AttnArgs a,
                                                           char* __restrict__ out, int64_t so_m, int64_t so_h) {
  const int rows = n_rep * M;   // query rows of this KV head's group
  constexpr int kSplitMin = RBW == 1 ? kHeadSplitMinSlots1 : kHeadSplitMinSlots2;
  __shared__ __attribute__((aligned(16))) HeadShared<RBW, W> lds;
  constexpr int ES = DTypeInfo<DT>::kSize;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int sp = (int)blockIdx.x;
  const int h = blockIdx.y;

  u32x4_t qf[RBW][kDSteps];
  int tok[RBW];
  bool row_ok[RBW];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    const int row = rb * 16 + r;
    row_ok[rb] = row < rows;
    const int i = row_ok[rb] ? row / (int)M : 0;
    tok[rb] = row_ok[rb] ? row % (int)M : 0;
    const char* qp = q + ((int64_t)tok[rb] * sq_m + (int64_t)(h * n_rep + i) * sq_h) * ES;
#pragma unroll
    for (int ds = 0; ds < kDSteps; ++ds) qf[rb][ds] = load16_sel(qp + (ds * 32 + 8 * g) * ES, row_ok[rb]);
  }
  const WaveKV<RBW> w = wave_kv<DT, RBW>(kc, vc, sh, head_bytes, a, h, tok, g, r);
  StepBuf<RBW> bA, bB;
  int c = (sp * W + wv) * kKeyStep;
  attn_load<DT, RBW>(a, w, c, bA);   // before the valid length is known
  float m_run[RBW], l_run[RBW];
  f32x4_t acc[RBW][kDTiles];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) acc[rb][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  int64_t lv = a.L_valid;
  if (lv_dev != nullptr) {
    const int64_t d = *lv_dev;
    lv = d < 0 ? 0 : (d < lv ? d : lv);
  }
  const int ce = (int)lv;
  // workgroups taking part: one up to kSplitMin valid slots, else enough for
  // a step per wave, at most the grid's; the others have nothing dealt
  const int S = (gridDim.x == 1 || ce <= kSplitMin)
                    ? 1
                    : min((int)gridDim.x, head_split(ce / kKeyStep + (ce % kKeyStep != 0), W));
  if (sp >= S) return;
  const int kStride = S * W * kKeyStep;
  // past ce the loads read stale slots or zeros: p = 0 and V zeroed
  while (c < ce) {
    attn_load<DT, RBW>(a, w, next_step(w, c + kStride, ce), bB);
    attn_step<DT, RBW>(a, qf, row_ok, bA, c, ce, g, m_run, l_run, acc);
    c += kStride;
    if (c >= ce) break;
    attn_load<DT, RBW>(a, w, next_step(w, c + kStride, ce), bA);
    attn_step<DT, RBW>(a, qf, row_ok, bB, c, ce, g, m_run, l_run, acc);
    c += kStride;
  }
  head_finish<DT, RBW, W>(lds, acc, m_run, l_run, a, sp, S, h, rows, M, n_rep, out, so_m, so_h);
}

// ------------------------------------ q/k norm + RoPE + cache write, fused
// The prologue of qkv_rope_cache_kernel inside the head form, for a forward
// whose M rows sit at the last M slots of the valid range [lv - M, lv) (the
// speculative runner's forwards): every wave norms and rotates its own query
// rows from the projection output as it loads them, and wave 0 of workgroup 0
// of each KV head norms and rotates the M new keys, writes them and the new
// values into the cache, and runs them as one extra 32-key step from
// registers and LDS.  The other steps cover the cached slots [0, lv - M) and
// are dealt exactly as in attn_head_kernel.  Rounding points as in
// qkv_rope_cache_kernel (the stock RMSNorm, then
// dtype(dtype(x * cos) + dtype(rotate_half(x) * sin))); only the order of the
// norm's fp32 sum of squares differs (per lane over its 32 dims, then across
// the head's four lanes).
struct RopeArgs {
  const char* qn;             // q_norm weight [D] or null
  const char* kn;             // k_norm weight [D] or null
  float eps;
  const char* cos;            // [n_pos, D] rows (stride scs)
  const char* sin;
  int64_t scs, n_pos;
  char* kcw;                  // the K / V tiles, written (the same as a.kc / a.vc)
  char* vcw;
  int Hq;
};

// The sum of one value per lane over the 16 lanes of a DPP row, the same fp32
// value on every lane: each stage pairs lanes symmetrically (lane xor 1, xor
// 2, then the half-row and row mirrors), and the add is commutative, so both
// partners form the same sum.
SIMSD_DEV float row16_sum(float v) {
  v += __int_as_float(dpp_quad_xor1(__float_as_int(v)));
  v += __int_as_float(dpp_quad_xor2(__float_as_int(v)));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));   // row_half_mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));   // row_mirror
  return v;
}

// Two values rounded to the dtype (bf16: one v_cvt_pk_bf16_f32, round to
// nearest even as the element-wise rounding), as packed bits and as floats.
template <int DT> SIMSD_DEV uint32_t pack_rnd2(float a, float b) { return pack2<DT>(a, b); }
template <int DT> SIMSD_DEV f32x2_t unpack2(uint32_t u) {
  return f32x2_t{h16_to_f32<DT>(u), h16_to_f32<DT>(u >> 16)};
}
template <int DT> SIMSD_DEV f32x2_t rnd2(float a, float b) { return unpack2<DT>(pack_rnd2<DT>(a, b)); }

// Norm + RoPE of one (token, head) row spread over the 16 lanes of a DPP row:
// lane j holds dims 8 j .. 8 j + 7 of x, of the norm weight w and of the cos
// / sin row c, s; the rotate_half partner of dim d < 64 is d + 64, held by
// lane j + 8, and back (one row rotation by 8).  Rounding points of
// qkv_rope_cache_kernel: w * dtype(x * r), rounded (the stock RMSNorm, r
// from the fp32 mean of squares), then dtype(dtype(x * cos) +
// dtype(rotate_half(x) * sin)); only the order of the fp32 sum of squares
// differs (per lane, then across the row).
template <int DT>
SIMSD_DEV u32x4_t norm_rope16(u32x4_t x, u32x4_t w, bool has_w, u32x4_t c, u32x4_t s, bool pos_ok, bool lower,
                              float eps) {
  const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
  f32x2_t xv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xv[i] = unpack2<DT>(xw[i]);
  uint32_t xn[4] = {xw[0], xw[1], xw[2], xw[3]};
  if (has_w) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ss += xv[i].x * xv[i].x;
      ss += xv[i].y * xv[i].y;
    }
    ss = row16_sum(ss);
    const float rr = 1.f / sqrtf(ss / (float)kHeadDim + eps);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2_t t = rnd2<DT>(xv[i].x * rr, xv[i].y * rr);
      const f32x2_t wf = unpack2<DT>(ww[i]);
      xn[i] = pack_rnd2<DT>(wf.x * t.x, wf.y * t.y);
      xv[i] = unpack2<DT>(xn[i]);
    }
  }
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w}, sw[4] = {s.x, s.y, s.z, s.w};
  uint32_t y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2_t pf = unpack2<DT>((uint32_t)dpp_row_ror8((int)xn[i]));   // the partner lane's values
    const f32x2_t cf = unpack2<DT>(cw[i]), sf = unpack2<DT>(sw[i]);
    const f32x2_t a = rnd2<DT>(xv[i].x * cf.x, xv[i].y * cf.y);
    const f32x2_t b = lower ? rnd2<DT>(-pf.x * sf.x, -pf.y * sf.y) : rnd2<DT>(pf.x * sf.x, pf.y * sf.y);
    y[i] = pos_ok ? pack_rnd2<DT>(a.x + b.x, a.y + b.y) : 0u;
  }
  return u32x4_t{y[0], y[1], y[2], y[3]};
}

constexpr int kNewKeysMax = 16;   // new rows of a fused forward (one 16-key tile)
constexpr int kTileStride = kHeadDim + 8;   // padded LDS rows of the q and K tiles (16-bit elements)

// grid (S_max + 1, Hkv) when S_max > 1 (one more workgroup per KV head: the
// new keys are one more dealt step), else (1, Hkv); W waves.
// qkv: the projection output [M, (Hq + 2 Hkv) * D] (row stride sqkv).
// Prologue: each (token, head) row of the projection output is a task of 16
// lanes (8 dims each) -- the rows * q rows of this KV head's group, then its
// M new keys and M new values -- dealt 4 to a wave pass; every workgroup
// norms and rotates its q rows into LDS, the workgroup that takes the new
// keys (below) its K into LDS and the cache and its V into LDS (transposed),
// then one workgroup barrier, and every wave reads its Q^T fragments.
// Steps: the new keys are step n_old = ceil((lv - M) / 32) in the head form's
// dealing (steps i < n_old are the cached 32-key steps), so the wave that gets
// them holds no cached step while the grid has a wave to spare; it writes the
// new V into the cache and runs the new keys' step from LDS.
// GATHERED: cos / sin hold the rows' own tables (row t at t * scs, gathered
// once per forward by the caller), so no row waits for its position before
// its cos / sin loads.
template <int DT, int RBW, int W, bool GATHERED>
__global__ __launch_bounds__(64 * W) void attn_head_rope_kernel(const char* __restrict__ qkv, const char* __restrict__ kc,
                                                                const char* __restrict__ vc,
                                                                const int64_t* __restrict__ lv_dev,
                                                                const int64_t* __restrict__ pos, int sqkv, int sh,
                                                                uint32_t head_bytes, int M, int n_rep, AttnArgs a,
                                                                RopeArgs ra, char* __restrict__ out, int64_t so_m,
                                                                int64_t so_h) {
  constexpr int MAXS = kHeadMaxSplit + 1;
  constexpr int ROWS = RBW * 16;
  constexpr int kPasses = (ROWS + 2 * kNewKeysMax + 4 * W - 1) / (4 * W);   // task passes per wave
  const int rows = n_rep * M;
  constexpr int kSplitMin = RBW == 1 ? kHeadSplitMinSlots1 : kHeadSplitMinSlots2;
  __shared__ __attribute__((aligned(16))) HeadShared<RBW, W, MAXS> lds;
  __shared__ __attribute__((aligned(16))) uint16_t q_t[ROWS][kTileStride];          // rotated q rows
  __shared__ __attribute__((aligned(16))) uint16_t k_t[kNewKeysMax][kTileStride];   // new K rows
  __shared__ __attribute__((aligned(16))) uint16_t vt_t[kHeadDim][32];              // new V, [dim][key]
  constexpr int ES = DTypeInfo<DT>::kSize;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int h = blockIdx.y;
  // role sp of this workgroup: workgroups go to the XCDs round robin by
  // linear id, so with an 8-wide grid the same role of every KV head -- the
  // new keys' owner among them -- would share one XCD; there the roles are
  // rotated by the head (1400 slots: 10.45 -> 10.06 us a layer; other widths
  // already spread them, and rotating 9 cost 2048 slots 0.2 us)
  const int sp = (gridDim.x & 7) == 0 ? (int)((blockIdx.x + gridDim.x - (unsigned)h % gridDim.x) % gridDim.x)
                                      : (int)blockIdx.x;

  // the rows' positions: scalar loads (uniform addresses, in bounds), or the
  // row index into pre-gathered tables
  int64_t pt[kNewKeysMax];
#pragma unroll
  for (int t = 0; t < kNewKeysMax; ++t) pt[t] = GATHERED ? t : pos[t < M ? t : 0];

  // this lane's tasks: task id = (pass * W + wave) * 4 + lane / 16, dims
  // 8 (lane % 16) ..; ids past the last task re-read task 0 and are dropped
  const int n_tasks = rows + 2 * M;
  const int jd = 8 * (lane & 15);
  int t_kind[kPasses], t_tok[kPasses];   // kind 0: q row, 1: new key, 2: new value, -1: none
  u32x4_t t_x[kPasses], t_w[kPasses];
  const char* qn_p = ra.qn != nullptr ? ra.qn : ra.cos;
  const char* kn_p = ra.kn != nullptr ? ra.kn : ra.cos;
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int t = (p * W + wv) * 4 + (lane >> 4);
    int kind = -1, tok = 0, head = 0;
    if (t < rows) {
      kind = 0; tok = t % M; head = h * n_rep + t / M;
    } else if (t < rows + M) {
      kind = 1; tok = t - rows; head = ra.Hq + h;
    } else if (t < n_tasks) {
      kind = 2; tok = t - rows - M; head = ra.Hq + a.Hkv + h;
    }
    t_kind[p] = kind;
    t_tok[p] = tok;
    t_x[p] = *reinterpret_cast<const u32x4_t*>(qkv + ((int64_t)tok * sqkv + (int64_t)head * kHeadDim + jd) * ES);
    t_w[p] = *reinterpret_cast<const u32x4_t*>((kind == 1 ? kn_p : qn_p) + jd * ES);
  }
  // the first cached step's K / V, before the valid length is known
  int tok_q[RBW];
  bool row_ok[RBW];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    const int row = rb * 16 + r;
    row_ok[rb] = row < rows;
    tok_q[rb] = row_ok[rb] ? row % M : 0;
  }
  const WaveKV<RBW> w = wave_kv<DT, RBW>(kc, vc, sh, head_bytes, a, h, tok_q, g, r);
  StepBuf<RBW> bA, bB;
  int c = (sp * W + wv) * kKeyStep;
  attn_load<DT, RBW>(a, w, c, bA);
  int64_t lv = a.L_valid;
  if (lv_dev != nullptr) {
    const int64_t d = *lv_dev;
    lv = d < 0 ? 0 : (d < lv ? d : lv);
  }
  const int ce = (int)lv;
  const int s0 = ce - M;   // the new rows' slots: [s0, ce)
  // cos / sin at each task's position
  u32x4_t t_c[kPasses], t_s[kPasses];
  bool t_pos_ok[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    int64_t pp = pt[0];
#pragma unroll
    for (int t = 1; t < kNewKeysMax; ++t) pp = t_tok[p] == t ? pt[t] : pp;
    t_pos_ok[p] = pp >= 0 && pp < ra.n_pos;
    const int64_t pr = t_pos_ok[p] ? pp : 0;
    t_c[p] = *reinterpret_cast<const u32x4_t*>(ra.cos + (pr * ra.scs + jd) * ES);
    t_s[p] = *reinterpret_cast<const u32x4_t*>(ra.sin + (pr * ra.scs + jd) * ES);
  }
  // the mask bytes of the new keys (columns s0 + 16 t + 4 g + j), a byte at a
  // time: s0 has any alignment
  uint8_t nmb[RBW][2][4];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    const uint8_t* mr = a.mask != nullptr ? a.mask + (int64_t)tok_q[rb] * a.smask
                                          : reinterpret_cast<const uint8_t*>(ra.cos);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = s0 + 16 * t + 4 * g + j;
        nmb[rb][t][j] = mr[k >= 0 && k < ce ? k : 0];
      }
  }
  // steps: the cached ones i < n_old, then the new keys as step n_old; step
  // i goes to workgroup (i / W) % S, wave i % W
  const int n_old = s0 > 0 ? (s0 + kKeyStep - 1) / kKeyStep : 0;
  const int S = (gridDim.x == 1 || ce <= kSplitMin)
                    ? 1
                    : min((int)gridDim.x, head_split(n_old + 1, W));
  if (sp >= S) return;
  const int new_wg = (n_old / W) % S;
  const bool owner = new_wg == sp && n_old % W == wv;
  char* kb = ra.kcw + (int64_t)h * sh * ES;
  char* vb = ra.vcw + (int64_t)h * sh * ES;
  // the tasks: q rows in every workgroup, the new keys and values in the one
  // that runs their step
  const bool lower = (lane & 15) < 8;   // dims below 64: partner d + 64
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int kind = t_kind[p], tok = t_tok[p];
    const int t = (p * W + wv) * 4 + (lane >> 4);
    if (kind == 0) {
      const u32x4_t y = norm_rope16<DT>(t_x[p], t_w[p], ra.qn != nullptr, t_c[p], t_s[p], t_pos_ok[p], lower, ra.eps);
      *reinterpret_cast<u32x4_t*>(&q_t[t][jd]) = y;
    } else if (kind == 1 && sp == new_wg) {
      const u32x4_t y = norm_rope16<DT>(t_x[p], t_w[p], ra.kn != nullptr, t_c[p], t_s[p], t_pos_ok[p], lower, ra.eps);
      *reinterpret_cast<u32x4_t*>(&k_t[tok][jd]) = y;
      const int64_t slot = (int64_t)s0 + tok;
      if (t_pos_ok[p] && slot >= 0 && slot < a.L_cap)
        *reinterpret_cast<u32x4_t*>(kb + k_tile_index(slot, jd) * ES) = y;
    } else if (kind == 2 && sp == new_wg) {
      const uint32_t vw[4] = {t_x[p].x, t_x[p].y, t_x[p].z, t_x[p].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) vt_t[jd + e][tok] = (uint16_t)(vw[e >> 1] >> (16 * (e & 1)));
    }
  }
  lds_barrier();
  u32x4_t qf[RBW][kDSteps];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb)
#pragma unroll
    for (int ds = 0; ds < kDSteps; ++ds) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&q_t[rb * 16 + r][ds * 32 + 8 * g]);
      qf[rb][ds] = row_ok[rb] ? v : zero4();
    }

  float m_run[RBW], l_run[RBW];
  f32x4_t acc[RBW][kDTiles];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) acc[rb][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  if (owner) {
    const bool key_ok = r < M;   // new key r = token r, lane row r
    StepBuf<RBW> bn;
#pragma unroll
    for (int ds = 0; ds < kDSteps; ++ds) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&k_t[r][ds * 32 + 8 * g]);
      bn.kf[0][ds] = key_ok ? v : zero4();
      bn.kf[1][ds] = zero4();
    }
    // keys past M hold stale LDS bits: the step zeroes their V and masks their
    // scores (they sit past ce)
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) {
      const int d = dt * 16 + r;
      const uint2 lo = *reinterpret_cast<const uint2*>(&vt_t[d][4 * g]);
      const uint2 hi = *reinterpret_cast<const uint2*>(&vt_t[d][16 + 4 * g]);
      bn.vf[dt] = u32x4_t{lo.x, lo.y, hi.x, hi.y};
    }
    // the new V into the cache: lane l takes dims l and l + 64 and, for each
    // quad of new keys, their 4 contiguous values in the V tile (slots
    // s0 + 4 q .. + 3 share a tile row when s0 % 4 == 0, the runner's case;
    // else one value at a time)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int d = lane + 64 * half;
      if ((s0 & 3) == 0) {
        for (int q4 = 0; q4 < (M + 3) / 4; ++q4) {
          const int64_t sq4 = (int64_t)s0 + 4 * q4;
          const int nk = min(4, M - 4 * q4);
          if (sq4 >= 0 && sq4 + 3 < a.L_cap && nk == 4) {
            *reinterpret_cast<uint2*>(vb + v_tile_index(sq4, d) * ES) =
                *reinterpret_cast<const uint2*>(&vt_t[d][4 * q4]);
          } else {
            for (int k = 0; k < nk; ++k)
              if (sq4 + k >= 0 && sq4 + k < a.L_cap)
                store_elem<DT>(vb, v_tile_index(sq4 + k, d), h16_to_f32<DT>(vt_t[d][4 * q4 + k]));
          }
        }
      } else {
        for (int k = 0; k < M; ++k)
          if ((int64_t)s0 + k >= 0 && (int64_t)s0 + k < a.L_cap)
            store_elem<DT>(vb, v_tile_index((int64_t)s0 + k, d), h16_to_f32<DT>(vt_t[d][k]));
      }
    }
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint32_t mw = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = s0 + 16 * t + 4 * g + j;
          const bool vis = a.mask == nullptr || nmb[rb][t][j] != 0;
          mw |= (k >= 0 && k < ce && vis ? 1u : 0u) << (8 * j);
        }
        bn.mk[rb][t] = mw;
      }
    attn_step<DT, RBW>(a, qf, row_ok, bn, s0, ce, g, m_run, l_run, acc);
  }
  // the cached slots [0, s0)
  const int kStride = S * W * kKeyStep;
  while (c < s0) {
    attn_load<DT, RBW>(a, w, next_step(w, c + kStride, s0), bB);
    attn_step<DT, RBW>(a, qf, row_ok, bA, c, s0, g, m_run, l_run, acc);
    c += kStride;
    if (c >= s0) break;
    attn_load<DT, RBW>(a, w, next_step(w, c + kStride, s0), bA);
    attn_step<DT, RBW>(a, qf, row_ok, bB, c, s0, g, m_run, l_run, acc);
    c += kStride;
  }
  head_finish<DT, RBW, W, MAXS>(lds, acc, m_run, l_run, a, sp, S, h, rows, M, n_rep, out, so_m, so_h);
}

constexpr int kMaxChunks = 1024;

// One workgroup per (token, query head), one thread per dim: merge the chunk
// partials in chunk order, normalise, round.  Rows with no visible key give 0.
// The chunk weights are formed once in LDS; the partial rows are read kBatch
// chunks at a time.
template <int DT>
__global__ __launch_bounds__(kHeadDim) void attn_combine_kernel(const float* __restrict__ o_part,
                                                               const float2* __restrict__ ml_part, int n_chunks,
                                                               int rows_pad, int64_t M, int Hq, int n_rep,
                                                               char* __restrict__ out, int64_t so_m, int64_t so_h,
                                                               const int64_t* __restrict__ lv_dev, int64_t chunk) {
  constexpr int kBatch = 8;
  const int64_t head_rows = (int64_t)n_chunks * rows_pad;   // partial rows per KV head
  // chunks past the device-side valid length were skipped: merge the others
  if (lv_dev != nullptr) {
    const int64_t v = *lv_dev;
    n_chunks = v <= 0 ? 0 : (int)min((int64_t)n_chunks, (v + chunk - 1) / chunk);
  }
  __shared__ float w_sh[kMaxChunks];
  __shared__ float red[kHeadDim / 64][2];
  const int64_t m = blockIdx.x / Hq;
  const int hq = blockIdx.x % Hq;
  const int h = hq / n_rep, i = hq % n_rep;
  const int64_t row = (int64_t)i * M + m;
  const int d = threadIdx.x;
  const int lane = d & 63, wv = d >> 6;
  const int64_t base = (int64_t)h * head_rows;
  // running maxima of the chunks: per thread over its chunks, then the block
  float mx = -INFINITY;
  for (int c = d; c < n_chunks; c += kHeadDim) {
    const float2 ml = ml_part[base + (int64_t)c * rows_pad + row];
    w_sh[c] = ml.x;
    mx = fmaxf(mx, ml.x);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wv][0] = mx;
  __syncthreads();
  mx = fmaxf(red[0][0], red[1][0]);
  // weights exp(m_c - max) and the denominator (each thread its chunks, then
  // the block in thread order)
  float l = 0.f;
  for (int c = d; c < n_chunks; c += kHeadDim) {
    const float mc = w_sh[c];
    const float wt = (mx == -INFINITY || mc == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mc - mx);
    w_sh[c] = wt;
    l += ml_part[base + (int64_t)c * rows_pad + row].y * wt;
  }
  l = wave_sum(l);
  if (lane == 0) red[wv][1] = l;
  __syncthreads();
  l = red[0][1] + red[1][1];
  float o = 0.f;
  for (int c0 = 0; c0 < n_chunks; c0 += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      v[u] = o_part[(base + (int64_t)min(c0 + u, n_chunks - 1) * rows_pad + row) * kHeadDim + d];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (c0 + u < n_chunks) o += v[u] * w_sh[c0 + u];
  }
  store_elem<DT>(out, m * so_m + (int64_t)hq * so_h + d, l > 0.f ? o / l : 0.f);
}

// ------------------------------------------------------ block visibility
// Attention mask rows of a cached forward over the slot space: [0, ctx_len)
// committed context, then from slot s0 the rows' own scratch slots in row
// order.  Rows: n_prefix rows of a committed block (folded in to store its
// K/V), n_free rows of the block being denoised, then K verify blocks of bl
// data rows and bl mask rows.  The verify rule is sdar/new_attn_multi_block.py:
// 22-183 on the layout of speculative_decoding/verify.py:350-418: data at
// position p carries step_map[k][p] + 1 (bs + 1, i.e. a mask, when never
// drafted), a mask token takes the step of the data token of equal
// within-block rank, and within a block
//   data i sees data j iff t_j <= t_i, mask j iff t_j > t_i,
//   mask i sees data j iff t_j <  t_i, mask j iff t_j >= t_i;
// a later block sees an earlier block's data only.  Every row sees the
// context and the prefix; the free block sees itself; nothing else is visible.
constexpr int kMaxVerifyTokens = 1024;

__global__ __launch_bounds__(256) void block_mask_kernel(uint8_t* __restrict__ mask, int64_t smask, int64_t n_cols,
                                                         int64_t ctx_len, int64_t s0, int n_prefix, int n_free, int K,
                                                         int bl, int bs, const int64_t* __restrict__ step_map) {
  __shared__ int8_t typ[kMaxVerifyTokens];      // 1 data, 2 mask
  __shared__ int16_t tim[kMaxVerifyTokens];
  const int nv = 2 * K * bl;
  auto label = [&](int v) {
    const int k = v / (2 * bl), w = v % (2 * bl);
    if (w >= bl) return bs + 1;
    const int64_t st = step_map[(int64_t)k * bl + w];
    return st >= 0 ? (int)st + 1 : bs + 1;
  };
  for (int v = threadIdx.x; v < nv; v += blockDim.x) {
    const int k = v / (2 * bl), w = v % (2 * bl);
    const int lab = label(v);
    const bool is_data = lab <= bs;
    int rank = 0;
    for (int u = 0; u < w; ++u) rank += ((label(k * 2 * bl + u) <= bs) == is_data) ? 1 : 0;
    int t = lab;
    if (!is_data) {   // the data token of the same rank, if any
      int seen = 0;
      for (int u = 0; u < 2 * bl; ++u) {
        const int lu = label(k * 2 * bl + u);
        if (lu <= bs) {
          if (seen == rank) { t = lu; break; }
          ++seen;
        }
      }
    }
    typ[v] = is_data ? 1 : 2;
    tim[v] = (int16_t)t;
  }
  __syncthreads();
  const int row = blockIdx.y;
  const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= n_cols) return;
  bool vis = false;
  if (col < ctx_len) {
    vis = true;
  } else if (col >= s0) {
    const int64_t u = col - s0;
    if (u < n_prefix) {
      // committed blocks: every later row sees them all; among themselves
      // block-causal, as when they are flushed into the cache one block at a
      // time (a row sees its own block and the ones before it)
      vis = row >= n_prefix || u / bl <= row / bl;
    } else if (u < n_prefix + n_free) {
      vis = row >= n_prefix && row < n_prefix + n_free;
    } else if (u < n_prefix + n_free + nv && row >= n_prefix + n_free) {
      const int j = (int)(u - n_prefix - n_free);
      const int i = row - n_prefix - n_free;
      const int ki = i / (2 * bl), kj = j / (2 * bl);
      if (ki == kj) {
        const int ti = tim[i], tj = tim[j];
        if (typ[i] == 1) vis = typ[j] == 1 ? tj <= ti : tj > ti;
        else vis = typ[j] == 1 ? tj < ti : tj >= ti;
      } else {
        vis = ki > kj && typ[j] == 1;
      }
    }
  }
  mask[(int64_t)row * smask + col] = vis ? 1 : 0;
}

struct AttnPlan {
  int rows, rows_pad, rb, rbw, waves, groups, n_chunks;
  bool ksplit, head;
  int split;                  // head form: workgroups per KV head
  int fsplit;                 // the same for the fused launch (qkv_rope_attention)
  int64_t chunk, wave_chunk;
  int64_t cnt_bytes, o_bytes, ml_bytes, bytes;
};

inline int64_t up256(int64_t n) { return (n + 255) / 256 * 256; }
inline int64_t up32(int64_t n) { return (n + 31) / 32 * 32; }

// Up to 32 query rows per KV head (two row blocks): four waves split each
// workgroup's key chunk, about 256 waves in all, at least one 32-key step per
// wave.  More rows: the row blocks spread over up to 4 waves (2 blocks per wave
// above 4 blocks) and row groups of 8 blocks, sharing 64-key or longer chunks.
AttnPlan attn_plan(int64_t M, int64_t Hq, int64_t Hkv, int64_t L_valid) {
  AttnPlan p{};
  const int n_rep = (int)(Hq / Hkv);
  p.rows = (int)(n_rep * M);
  p.rb = (p.rows + 15) / 16;
  p.rows_pad = p.rb * 16;
  const int64_t L = L_valid > 0 ? L_valid : 1;
  p.ksplit = p.rb <= 2;
  if (p.ksplit) {
    p.rbw = p.rb;
    p.waves = 4;
    p.groups = 1;
    int64_t wc = up32((Hkv * L + 255) / 256);            // keys per wave for ~256 waves
    if (wc < 32) wc = 32;
    while ((L + 4 * wc - 1) / (4 * wc) > kMaxChunks) wc *= 2;
    p.wave_chunk = wc;
    p.chunk = 4 * wc;
  } else {
    // up to 8 row blocks: one a wave, in row groups of at most 4 waves
    // (8 blocks: two groups of 4, 19.4 -> 17.3 us a layer against 4 waves of
    // two blocks); more: two blocks a wave, in as few groups of at most 4
    // waves as hold them, balanced (9 blocks: two groups of 3 waves rather
    // than 8 blocks and 1)
    if (p.rb <= 8) {
      p.rbw = 1;
      p.groups = (p.rb + 3) / 4;
      p.waves = (p.rb + p.groups - 1) / p.groups;
    } else {
      p.rbw = 2;
      p.groups = (p.rb + 7) / 8;
      p.waves = ((p.rb + p.groups - 1) / p.groups + 1) / 2;
    }
    int64_t want = (256 + Hkv - 1) / Hkv;                  // chunks per head
    int64_t chunk = (L + want - 1) / want;
    chunk = (chunk + 63) / 64 * 64;
    if (chunk < 64) chunk = 64;
    while ((L + chunk - 1) / chunk > kMaxChunks) chunk *= 2;
    p.chunk = chunk;
    p.wave_chunk = chunk;
  }
  p.n_chunks = (int)((L + p.chunk - 1) / p.chunk);
  p.head = p.ksplit && L <= kHeadMaxSlots;   // one launch
  // head form: the grid holds the workgroups the bound L could use; the
  // kernel takes as many as the device-side length needs
  p.split = 1;
  p.fsplit = 1;
  if (p.head && L > (p.rbw == 2 ? kHeadSplitMinSlots2 : kHeadSplitMinSlots1)) {
    const int W = p.rbw == 2 ? kHeadW2 : kHeadW1;
    const int steps = (int)((L + kKeyStep - 1) / kKeyStep);
    // the most any valid length up to L asks for: head_split drops where it
    // switches to 1.5 steps a wave (28 steps: 7 workgroups, 29: 5)
    auto most = [&](int n) { return std::max(head_split(n, W), head_split(std::min(n, SIMSD_HEAD_SPW_SWITCH), W)); };
    p.split = std::min(kHeadMaxSplit, most(steps));
    // the fused launch: its new keys are one more step after the cached ones
    // (at most the steps of L, plus one)
    p.fsplit = std::min(kHeadMaxSplit + 1, most(steps + 1));
  }
  // workspace: [arrival counters][o partials][(max, sum) partials]; the
  // counters come first in every form so that a workspace shared between
  // calls keeps them at zero
  // the head form's partials: split, or fsplit in the fused launch (its new
  // keys may take one more workgroup), whichever call uses the workspace
  const int64_t parts = p.head ? std::max(p.split, p.fsplit) : p.n_chunks;
  p.cnt_bytes = up256(Hkv * 4);
  p.o_bytes = up256(Hkv * parts * p.rows_pad * kHeadDim * 4);
  p.ml_bytes = up256(Hkv * parts * p.rows_pad * 8);
  p.bytes = (p.head && p.split == 1) ? 0 : p.cnt_bytes + p.o_bytes + p.ml_bytes;
  return p;
}

inline bool al(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

}  // namespace
}  // namespace simsd

using namespace simsd;

extern "C" int simsd_qkv_rope_cache(const void* qkv, int64_t sqkv, const void* q_norm_w, const void* k_norm_w,
                                    float eps, const void* cos, const void* sin, int64_t scs, int64_t n_pos,
                                    const int64_t* pos, const int64_t* slots, const int64_t* slots2, void* k_cache,
                                    void* v_cache, int64_t kv_head_stride, int64_t L, void* q_out, int64_t sqo_m,
                                    int64_t sqo_h, int64_t M, int64_t Hq, int64_t Hkv, int64_t head_dim, int dtype,
                                    void* stream) {
  if (dtype != kBF16 && dtype != kF16) return set_error("qkv_rope_cache: dtype must be bf16 or fp16");
  if (head_dim != kHeadDim) return set_error("qkv_rope_cache: head_dim must be %d (got %lld)", kHeadDim, (long long)head_dim);
  if (M < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || L <= 0 || n_pos <= 0)
    return set_error("qkv_rope_cache: bad sizes");
  if (L % 32 != 0 || kv_head_stride < L * kHeadDim)
    return set_error("qkv_rope_cache: the cache needs L %% 32 == 0 and a head stride of at least L * %d", kHeadDim);
  if (M == 0) return 0;
  if (M > 0x7fffffff) return set_error("qkv_rope_cache: too many tokens");
  if (sqkv < 0 || sqkv > 0x7fffffff) return set_error("qkv_rope_cache: row stride out of range");
  if (!qkv || !cos || !sin || !pos || !slots || !k_cache || !v_cache || !q_out)
    return set_error("qkv_rope_cache: null pointer");
  QkvArgs a{};
  a.qkv = static_cast<const char*>(qkv); a.sqkv = sqkv;
  a.qn = static_cast<const char*>(q_norm_w); a.kn = static_cast<const char*>(k_norm_w); a.eps = eps;
  a.cos = static_cast<const char*>(cos); a.sin = static_cast<const char*>(sin); a.scs = scs; a.n_pos = n_pos;
  a.pos = pos; a.slots = slots; a.slots2 = slots2;
  a.kc = static_cast<char*>(k_cache); a.vc = static_cast<char*>(v_cache); a.sh = kv_head_stride; a.L = L;
  a.qo = static_cast<char*>(q_out); a.sqo_m = sqo_m; a.sqo_h = sqo_h;
  a.Hq = (int)Hq; a.Hkv = (int)Hkv;
  const int heads = (int)(Hq + 2 * Hkv);
  const int waves = heads < 8 ? heads : 8;
  const dim3 grid((unsigned)M, (unsigned)((heads + waves - 1) / waves));
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto kern = dtype == kBF16 ? qkv_rope_cache_kernel<kBF16, false> : qkv_rope_cache_kernel<kF16, false>;
  hipLaunchKernelGGL(kern, grid, dim3(64 * waves), 0, st, a.qkv, a.pos, a.slots, a.qn, a.kn, (int)a.sqkv, a.Hq,
                     a.Hkv, a);
  return check_launch("qkv_rope_cache");
}

extern "C" int simsd_reduce_qkv_rope_cache(const void* part, int split, int64_t part_bytes, const void* q_norm_w,
                                           const void* k_norm_w, float eps, const void* cos, const void* sin,
                                           int64_t scs, int64_t n_pos, const int64_t* pos, const int64_t* slots,
                                           const int64_t* slots2, void* k_cache, void* v_cache,
                                           int64_t kv_head_stride, int64_t L, void* q_out, int64_t sqo_m,
                                           int64_t sqo_h, int64_t M, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                           int dtype, void* stream) {
  if (dtype != kBF16 && dtype != kF16) return set_error("reduce_qkv_rope_cache: dtype must be bf16 or fp16");
  if (head_dim != kHeadDim)
    return set_error("reduce_qkv_rope_cache: head_dim must be %d (got %lld)", kHeadDim, (long long)head_dim);
  if (M < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || L <= 0 || n_pos <= 0)
    return set_error("reduce_qkv_rope_cache: bad sizes");
  if (split < 1 || split > kQkvMaxSplit)
    return set_error("reduce_qkv_rope_cache: split must be 1..%d (got %d)", kQkvMaxSplit, split);
  if (L % 32 != 0 || kv_head_stride < L * kHeadDim)
    return set_error("reduce_qkv_rope_cache: the cache needs L %% 32 == 0 and a head stride of at least L * %d",
                     kHeadDim);
  if (M == 0) return 0;
  if (M > 0x7fffffff) return set_error("reduce_qkv_rope_cache: too many tokens");
  const int64_t N = (Hq + 2 * Hkv) * kHeadDim;
  if (part_bytes < (int64_t)split * M * N * 4)
    return set_error("reduce_qkv_rope_cache: %d partials of %lld x %lld need %lld bytes (got %lld)", split,
                     (long long)M, (long long)N, (long long)split * M * N * 4, (long long)part_bytes);
  if (!part || !cos || !sin || !pos || !slots || !k_cache || !v_cache || !q_out)
    return set_error("reduce_qkv_rope_cache: null pointer");
  QkvArgs a{};
  a.qkv = nullptr; a.sqkv = N;
  a.part = static_cast<const float*>(part); a.split = split; a.part_mn = M * N;
  a.qn = static_cast<const char*>(q_norm_w); a.kn = static_cast<const char*>(k_norm_w); a.eps = eps;
  a.cos = static_cast<const char*>(cos); a.sin = static_cast<const char*>(sin); a.scs = scs; a.n_pos = n_pos;
  a.pos = pos; a.slots = slots; a.slots2 = slots2;
  a.kc = static_cast<char*>(k_cache); a.vc = static_cast<char*>(v_cache); a.sh = kv_head_stride; a.L = L;
  a.qo = static_cast<char*>(q_out); a.sqo_m = sqo_m; a.sqo_h = sqo_h;
  a.Hq = (int)Hq; a.Hkv = (int)Hkv;
  const int heads = (int)(Hq + 2 * Hkv);
  const int waves = heads < 8 ? heads : 8;
  const dim3 grid((unsigned)M, (unsigned)((heads + waves - 1) / waves));
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto kern = dtype == kBF16 ? qkv_rope_cache_kernel<kBF16, true> : qkv_rope_cache_kernel<kF16, true>;
  hipLaunchKernelGGL(kern, grid, dim3(64 * waves), 0, st, a.qkv, a.pos, a.slots, a.qn, a.kn, (int)a.sqkv, a.Hq,
                     a.Hkv, a);
  return check_launch("reduce_qkv_rope_cache");
}

extern "C" int64_t simsd_block_attention_workspace_bytes(int64_t M, int64_t Hq, int64_t Hkv, int64_t L_valid) {
  if (M < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || L_valid < 0) return -1;
  return attn_plan(M, Hq, Hkv, L_valid).bytes;
}

extern "C" int simsd_block_attention(const void* q, int64_t sq_m, int64_t sq_h, const void* k_cache,
                                     const void* v_cache, int64_t kv_head_stride, int64_t L_cap,
                                     const uint8_t* mask, int64_t smask, void* out, int64_t so_m, int64_t so_h,
                                     int64_t M, int64_t Hq, int64_t Hkv, int64_t L_valid,
                                     const int64_t* valid_len_dev, int64_t head_dim, float scale, int dtype,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  if (dtype != kBF16 && dtype != kF16) return set_error("block_attention: dtype must be bf16 or fp16");
  if (head_dim != kHeadDim) return set_error("block_attention: head_dim must be %d (got %lld)", kHeadDim, (long long)head_dim);
  if (M < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || L_valid < 0 || L_valid > L_cap)
    return set_error("block_attention: bad sizes (M=%lld Hq=%lld Hkv=%lld L_valid=%lld L_cap=%lld)", (long long)M,
                     (long long)Hq, (long long)Hkv, (long long)L_valid, (long long)L_cap);
  if (M == 0) return 0;
  if (L_cap % 32 != 0 || kv_head_stride < L_cap * kHeadDim)
    return set_error("block_attention: the cache needs L_cap %% 32 == 0 and a head stride of at least L_cap * %d",
                     kHeadDim);
  if (L_cap * kHeadDim * 2 > (int64_t)0xFFFF0000) return set_error("block_attention: L_cap too large");   // step offsets past it stay below 2^32
  if (!q || !k_cache || !v_cache || !out) return set_error("block_attention: null pointer");
  if (sq_m < 0 || sq_m > 0x7fffffff || sq_h < 0 || sq_h > 0x7fffffff || kv_head_stride > 0x7fffffff)
    return set_error("block_attention: strides must fit 31 bits");   // 32-bit kernel arguments
  const AttnPlan pl = attn_plan(M, Hq, Hkv, L_valid);
  if (pl.rows > 65536) return set_error("block_attention: %d query rows per KV head exceed 65536", pl.rows);
  // 16-byte loads of q rows and of the K / V tiles
  if (!al(q, 16) || (sq_m % 8) || (sq_h % 8) || !al(k_cache, 16) || !al(v_cache, 16) || (kv_head_stride % 8))
    return set_error("block_attention: q rows and the K / V tiles must be 16-byte aligned");
  if (mask != nullptr && (!al(mask, 4) || smask % 4 != 0 || smask < (L_valid + 3) / 4 * 4))
    return set_error("block_attention: mask rows must be 4-byte aligned with at least L_valid rounded up to 4 bytes");
  if (pl.bytes > 0 && (workspace == nullptr || workspace_bytes < pl.bytes || !al(workspace, 16)))
    return set_error("block_attention: needs a 16-byte aligned workspace of %lld bytes (got %lld)", (long long)pl.bytes,
                     (long long)workspace_bytes);
  AttnArgs a{};
  a.q = static_cast<const char*>(q); a.sq_m = sq_m; a.sq_h = sq_h;
  a.kc = static_cast<const char*>(k_cache); a.vc = static_cast<const char*>(v_cache);
  a.sh = kv_head_stride; a.L_cap = L_cap;
  a.mask = mask; a.smask = smask;
  a.lv_dev = valid_len_dev;
  a.M = M; a.n_rep = (int)(Hq / Hkv); a.Hkv = (int)Hkv;
  a.L_valid = L_valid; a.chunk = pl.chunk; a.wave_chunk = pl.wave_chunk; a.n_chunks = pl.n_chunks;
  a.scale = scale;
  a.rows = pl.rows; a.rows_pad = pl.rows_pad;
  a.arrivals = static_cast<unsigned*>(workspace);
  a.o_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.cnt_bytes);
  a.ml_part = reinterpret_cast<float2*>(static_cast<char*>(workspace) + pl.cnt_bytes + pl.o_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)pl.n_chunks, (unsigned)Hkv, (unsigned)pl.groups), block(64 * pl.waves);
  auto partial = [&](auto dt_tag) {
    constexpr int DT = decltype(dt_tag)::value;
    if (pl.head) {
      char* o = static_cast<char*>(out);
      const dim3 hgrid((unsigned)pl.split, (unsigned)Hkv);
      const uint32_t head_bytes = (uint32_t)(L_cap * kHeadDim * 2);
      if (pl.rbw == 2)
        hipLaunchKernelGGL((attn_head_kernel<DT, 2, kHeadW2>), hgrid, dim3(64 * kHeadW2), 0, st, a.q, a.kc, a.vc,
                           a.lv_dev, (int)a.sq_m, (int)a.sq_h, (int)a.sh, head_bytes, (int)a.M, a.n_rep, a, o, so_m,
                           so_h);
      else
        hipLaunchKernelGGL((attn_head_kernel<DT, 1, kHeadW1>), hgrid, dim3(64 * kHeadW1), 0, st, a.q, a.kc, a.vc,
                           a.lv_dev, (int)a.sq_m, (int)a.sq_h, (int)a.sh, head_bytes, (int)a.M, a.n_rep, a, o, so_m,
                           so_h);
      return;
    }
    if (pl.ksplit) {
      if (pl.rbw == 2) hipLaunchKernelGGL((attn_partial_kernel<DT, 2, true>), grid, block, 0, st, a);
      else hipLaunchKernelGGL((attn_partial_kernel<DT, 1, true>), grid, block, 0, st, a);
    } else {
      if (pl.rbw == 2) hipLaunchKernelGGL((attn_partial_kernel<DT, 2, false>), grid, block, 0, st, a);
      else hipLaunchKernelGGL((attn_partial_kernel<DT, 1, false>), grid, block, 0, st, a);
    }
    hipLaunchKernelGGL(attn_combine_kernel<DT>, dim3((unsigned)(M * Hq)), dim3(kHeadDim), 0, st, a.o_part,
                       a.ml_part, pl.n_chunks, pl.rows_pad, M, (int)Hq, a.n_rep, static_cast<char*>(out), so_m, so_h,
                       a.lv_dev, pl.chunk);
  };
  if (dtype == kBF16) partial(std::integral_constant<int, kBF16>{});
  else partial(std::integral_constant<int, kF16>{});
  return check_launch("block_attention");
}

extern "C" int simsd_qkv_rope_attention(const void* qkv, int64_t sqkv, const void* q_norm_w, const void* k_norm_w,
                                        float eps, const void* cos, const void* sin, int64_t scs, int64_t n_pos,
                                        const int64_t* pos, void* k_cache, void* v_cache, int64_t kv_head_stride,
                                        int64_t L_cap, const uint8_t* mask, int64_t smask, void* out, int64_t so_m,
                                        int64_t so_h, int64_t M, int64_t Hq, int64_t Hkv, int64_t L_valid,
                                        const int64_t* valid_len_dev, int64_t head_dim, float scale, int dtype,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  if (dtype != kBF16 && dtype != kF16) return set_error("qkv_rope_attention: dtype must be bf16 or fp16");
  if (head_dim != kHeadDim)
    return set_error("qkv_rope_attention: head_dim must be %d (got %lld)", kHeadDim, (long long)head_dim);
  if (M < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || L_valid < 0 || L_valid > L_cap || n_pos <= 0)
    return set_error("qkv_rope_attention: bad sizes (M=%lld Hq=%lld Hkv=%lld L_valid=%lld L_cap=%lld)",
                     (long long)M, (long long)Hq, (long long)Hkv, (long long)L_valid, (long long)L_cap);
  if (M == 0) return 0;
  if (M > kNewKeysMax) return set_error("qkv_rope_attention: at most %d rows (got %lld)", kNewKeysMax, (long long)M);
  if (L_cap % 32 != 0 || kv_head_stride < L_cap * kHeadDim)
    return set_error("qkv_rope_attention: the cache needs L_cap %% 32 == 0 and a head stride of at least L_cap * %d",
                     kHeadDim);
  if (L_cap * kHeadDim * 2 > (int64_t)0xFFFF0000) return set_error("qkv_rope_attention: L_cap too large");
  if (!qkv || !cos || !sin || !k_cache || !v_cache || !out)
    return set_error("qkv_rope_attention: null pointer");
  if (pos == nullptr && n_pos < M)
    return set_error("qkv_rope_attention: without positions, cos / sin must hold the %lld rows' tables",
                     (long long)M);
  if (sqkv < (Hq + 2 * Hkv) * kHeadDim || sqkv > 0x7fffffff || kv_head_stride > 0x7fffffff)
    return set_error("qkv_rope_attention: strides out of range");
  // 16-byte loads of the projection rows, the norm weights and the cos / sin
  // rows, 16-byte K tile stores
  if (!al(qkv, 16) || sqkv % 8 || !al(cos, 16) || !al(sin, 16) || scs % 8 || !al(k_cache, 16) ||
      !al(v_cache, 16) || kv_head_stride % 8 || (q_norm_w && !al(q_norm_w, 16)) || (k_norm_w && !al(k_norm_w, 16)))
    return set_error("qkv_rope_attention: operands must be 16-byte aligned");
  if (mask != nullptr && (smask < (L_valid + 3) / 4 * 4 || smask % 4 != 0 || !al(mask, 4)))
    return set_error("qkv_rope_attention: mask rows must be 4-byte aligned with at least L_valid rounded up to 4 bytes");
  const AttnPlan pl = attn_plan(M, Hq, Hkv, L_valid);
  if (!pl.head) return set_error("qkv_rope_attention: %d rows per KV head over %lld slots need the chunked form "
                                 "(qkv_rope_cache, then block_attention)", pl.rows, (long long)L_valid);
  if (pl.bytes > 0 && (workspace == nullptr || workspace_bytes < pl.bytes || !al(workspace, 16)))
    return set_error("qkv_rope_attention: needs a 16-byte aligned workspace of %lld bytes (got %lld)",
                     (long long)pl.bytes, (long long)workspace_bytes);
  AttnArgs a{};
  a.kc = static_cast<const char*>(k_cache); a.vc = static_cast<const char*>(v_cache);
  a.sh = kv_head_stride; a.L_cap = L_cap;
  a.mask = mask; a.smask = smask;
  a.lv_dev = valid_len_dev;
  a.M = M; a.n_rep = (int)(Hq / Hkv); a.Hkv = (int)Hkv;
  a.L_valid = L_valid; a.chunk = pl.chunk; a.wave_chunk = pl.wave_chunk; a.n_chunks = pl.n_chunks;
  a.scale = scale;
  a.rows = pl.rows; a.rows_pad = pl.rows_pad;
  a.arrivals = static_cast<unsigned*>(workspace);
  a.o_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.cnt_bytes);
  a.ml_part = reinterpret_cast<float2*>(static_cast<char*>(workspace) + pl.cnt_bytes + pl.o_bytes);
  RopeArgs ra{};
  ra.qn = static_cast<const char*>(q_norm_w); ra.kn = static_cast<const char*>(k_norm_w); ra.eps = eps;
  ra.cos = static_cast<const char*>(cos); ra.sin = static_cast<const char*>(sin); ra.scs = scs; ra.n_pos = n_pos;
  ra.kcw = static_cast<char*>(k_cache); ra.vcw = static_cast<char*>(v_cache);
  ra.Hq = (int)Hq;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the fused grid: the new keys are one more dealt step
  const dim3 hgrid((unsigned)pl.fsplit, (unsigned)Hkv);
  const uint32_t head_bytes = (uint32_t)(L_cap * kHeadDim * 2);
  const char* x = static_cast<const char*>(qkv);
  char* o = static_cast<char*>(out);
  auto go = [&](auto dt_tag, auto g_tag) {
    constexpr int DT = decltype(dt_tag)::value;
    constexpr bool G = decltype(g_tag)::value;
    if (pl.rbw == 2)
      hipLaunchKernelGGL((attn_head_rope_kernel<DT, 2, kHeadW2, G>), hgrid, dim3(64 * kHeadW2), 0, st, x, a.kc,
                         a.vc, a.lv_dev, pos, (int)sqkv, (int)a.sh, head_bytes, (int)a.M, a.n_rep, a, ra, o, so_m,
                         so_h);
    else
      hipLaunchKernelGGL((attn_head_rope_kernel<DT, 1, kHeadW1, G>), hgrid, dim3(64 * kHeadW1), 0, st, x, a.kc,
                         a.vc, a.lv_dev, pos, (int)sqkv, (int)a.sh, head_bytes, (int)a.M, a.n_rep, a, ra, o, so_m,
                         so_h);
  };
  using gathered = std::integral_constant<bool, true>;
  using by_pos = std::integral_constant<bool, false>;
  if (dtype == kBF16) {
    if (pos == nullptr) go(std::integral_constant<int, kBF16>{}, gathered{});
    else go(std::integral_constant<int, kBF16>{}, by_pos{});
  } else {
    if (pos == nullptr) go(std::integral_constant<int, kF16>{}, gathered{});
    else go(std::integral_constant<int, kF16>{}, by_pos{});
  }
  return check_launch("qkv_rope_attention");
}

extern "C" int simsd_block_mask(uint8_t* mask, int64_t smask, int64_t n_cols, int64_t ctx_len, int64_t s0,
                                int n_prefix, int n_free, int K, int bl, int bs, const int64_t* step_map,
                                void* stream) {
  if (mask == nullptr || n_cols <= 0 || smask < n_cols || ctx_len < 0 || s0 < ctx_len || n_prefix < 0 ||
      n_free < 0 || K < 0 || bl <= 0 || bs <= 0 || bs > 30000)
    return set_error("block_mask: bad arguments");
  if (2LL * K * bl > kMaxVerifyTokens) return set_error("block_mask: more than %d verify tokens", kMaxVerifyTokens);
  if (K > 0 && step_map == nullptr) return set_error("block_mask: null step_map");
  const int64_t rows = n_prefix + n_free + 2LL * K * bl;
  if (rows == 0) return 0;
  if (rows > 65535) return set_error("block_mask: too many rows");
  if (s0 + n_prefix + n_free + 2LL * K * bl > n_cols) return set_error("block_mask: scratch slots past n_cols");
  const dim3 grid((unsigned)((n_cols + 255) / 256), (unsigned)rows);
  hipLaunchKernelGGL(block_mask_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), mask, smask, n_cols,
                     ctx_len, s0, n_prefix, n_free, K, bl, bs, step_map);
  return check_launch("block_mask");
}

// Batch-1 weight-only GEMV for gfx950.
//
// Replaces the reference's weight-only matvec family
// (src/kernels/kernels_weight_only_matvec.cu:60-133,359-436 W8A16/W4A16,
// :137-357,438-635 dp4a tiles) and the fp16 projection GEMV
// (src/kernels/kernels_ops_matvec.cu:343-418), plus the norm / RoPE / KV-store /
// residual / SiLU launches that surround them in the decode step
// (src/engine/llama_engine_graph.cpp:166-480).
//
// Design (MI355X):
//  * Weights stay in the reference's row-major layout; a wave covers 8 rows x
//    8 sixteen-byte chunks, so each row contributes 128 contiguous bytes per
//    step and every lane issues one 128-bit load per step.
//  * The activation vector is converted once per workgroup into a "prepared"
//    fp16 form in LDS so the inner loop needs no conversion instructions:
//    a packed weight dword is turned into two fp16 lanes by OR-ing its nibbles
//    (or bytes) under the exponent of 1024.0 and is consumed by v_dot2_f32_f16
//    with fp32 accumulation.  The bias that the exponent trick introduces is a
//    per-chunk constant of x and is pre-subtracted (the dot chain starts at
//    -C).  High nibbles land at 16x weight, which is compensated by storing
//    x/16 for those lanes (exact power-of-two scaling).
//  * fp16 weights are dotted against a hi/lo split of the fp32 activation so the
//    product keeps ~22 bits of the activation.
//  * Optional RMSNorm prologue (statistics in fp32) and fused epilogues
//    (residual add, SwiGLU, RoPE + KV-cache store) remove the small launches.
#include <cstdlib>

#include "common.hpp"
#include "gemv_plan.hpp"
#include "../../include/cpi_hip.h"

namespace cpi {

constexpr int kBlock = kWave * kWavesPerBlock;
static_assert(kTileRows * kChunkCols == kWave, "a wave covers 8 rows x 8 chunks");

template <int FMT> struct FmtT;
template <> struct FmtT<CPI_W_F16> {
  static constexpr int kElems = 8;    // fp16 per 16-byte chunk
  static constexpr int kStride = 8;   // LDS dwords per chunk: 4 hi + 4 lo
};
template <> struct FmtT<CPI_W_I8ROW> {
  static constexpr int kElems = 16;
  static constexpr int kStride = 12;  // 8 pair dwords + -C, padded to 16 B
};
template <> struct FmtT<CPI_W_I4ROW> {
  static constexpr int kElems = 32;
  static constexpr int kStride = 20;  // 16 pair dwords + -C, padded to 16 B
};
template <> struct FmtT<CPI_W_I4G32> : FmtT<CPI_W_I4ROW> {};

struct GemvParams {
  const void* w;
  const void* scales;
  int scale_count;
  int R, K;
  const void* x;
  const uint16_t* norm_w;
  float eps;
  void* y;
  void* y2;        // second output (dual GEMV, fp16)
  int rows_a;      // dual: rows belonging to output y (rest go to y2)
  int nh, nkv, hd;
  const int* position;
  const float* rope_cos;
  const float* rope_sin;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int max_ctx;
};

enum { EPI_DUAL_F16 = 100 };

// Workgroup barrier that only orders LDS: waits for this wave's LDS operations
// (lgkmcnt) but leaves outstanding global loads in flight, unlike
// __syncthreads(), whose fence drains them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt=63 (no wait), expcnt=7, lgkmcnt=0
  __builtin_amdgcn_s_barrier();
}

// ---------------------------------------------------------------------------
// Activation preparation (one chunk).
// ---------------------------------------------------------------------------
template <int FMT>
__device__ __forceinline__ void prep_chunk(const float* v, uint32_t* dst) {
  if constexpr (FMT == CPI_W_F16) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const f16 h0 = static_cast<f16>(v[2 * d]);
      const f16 h1 = static_cast<f16>(v[2 * d + 1]);
      const f16 l0 = static_cast<f16>(v[2 * d] - static_cast<float>(h0));
      const f16 l1 = static_cast<f16>(v[2 * d + 1] - static_cast<float>(h1));
      dst[d] = h2_bits(h0, h1);
      dst[4 + d] = h2_bits(l0, l1);
    }
  } else if constexpr (FMT == CPI_W_I8ROW) {
    // byte b' = q + 128 sits under 1024.0:  h = 1152 + q.
    float asum = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const f16 a0 = static_cast<f16>(v[4 * d + 0]);
      const f16 a1 = static_cast<f16>(v[4 * d + 1]);
      const f16 a2 = static_cast<f16>(v[4 * d + 2]);
      const f16 a3 = static_cast<f16>(v[4 * d + 3]);
      dst[2 * d + 0] = h2_bits(a0, a2);
      dst[2 * d + 1] = h2_bits(a1, a3);
      asum += (static_cast<float>(a0) + static_cast<float>(a1)) +
              (static_cast<float>(a2) + static_cast<float>(a3));
    }
    dst[8] = __builtin_bit_cast(uint32_t, -1152.f * asum);
  } else {
    // nibble n' = q + 8.  Low nibbles: h = 1024 + n', paired with a = x.
    // High nibbles: h = 1024 + 16 n', paired with a = x/16.
    // sum h*a = 1024*sum(a) + sum(n' * x~) with x~ = 16a on high lanes, so
    // sum(q x~) = sum(h a) - [1024*sum(a) + 8*sum(x~)].
    float c = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float* e = v + 8 * d;
      const f16 p0 = static_cast<f16>(e[0]), p4 = static_cast<f16>(e[4]);
      const f16 p1 = static_cast<f16>(e[1] * 0.0625f), p5 = static_cast<f16>(e[5] * 0.0625f);
      const f16 p2 = static_cast<f16>(e[2]), p6 = static_cast<f16>(e[6]);
      const f16 p3 = static_cast<f16>(e[3] * 0.0625f), p7 = static_cast<f16>(e[7] * 0.0625f);
      dst[4 * d + 0] = h2_bits(p0, p4);
      dst[4 * d + 1] = h2_bits(p1, p5);
      dst[4 * d + 2] = h2_bits(p2, p6);
      dst[4 * d + 3] = h2_bits(p3, p7);
      const float lo = (static_cast<float>(p0) + static_cast<float>(p4)) +
                       (static_cast<float>(p2) + static_cast<float>(p6));
      const float hi = (static_cast<float>(p1) + static_cast<float>(p5)) +
                       (static_cast<float>(p3) + static_cast<float>(p7));
      c += 1024.f * (lo + hi) + 8.f * (lo + 16.f * hi);
    }
    dst[16] = __builtin_bit_cast(uint32_t, -c);
  }
}

// ---------------------------------------------------------------------------
// Dot of one 16-byte weight chunk with its prepared activations.
// ---------------------------------------------------------------------------
template <int FMT>
__device__ __forceinline__ float chunk_dot(const u32x4 w, const uint32_t* p, float acc) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
  if constexpr (FMT == CPI_W_F16) {
    const uint4 ph = *reinterpret_cast<const uint4*>(p);
    const uint4 pl = *reinterpret_cast<const uint4*>(p + 4);
    const uint32_t h[4] = {ph.x, ph.y, ph.z, ph.w};
    const uint32_t l[4] = {pl.x, pl.y, pl.z, pl.w};
    float t[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) t[d] = dot2(wd[d], l[d], dot2(wd[d], h[d], 0.f));
    return acc + ((t[0] + t[1]) + (t[2] + t[3]));
  } else if constexpr (FMT == CPI_W_I8ROW) {
    // (w ^ 0x80808080) & 0x00FF00FF | 0x64006400 == (w & 0x00FF00FF) ^ 0x64806480
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    const uint32_t pp[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float t[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
      t[d] = dot2(((wd[d] >> 8) & 0x00FF00FFu) ^ 0x64806480u, pp[2 * d + 1],
                  dot2((wd[d] & 0x00FF00FFu) ^ 0x64806480u, pp[2 * d], 0.f));
    return acc + (((t[0] + t[1]) + (t[2] + t[3])) + __builtin_bit_cast(float, p[8]));
  } else {
    // Two's complement nibble n -> offset binary n ^ 8, placed under the
    // exponent of 1024.0:  (w & M) ^ (0x6400 | 8<<shift) per half.
    uint32_t pp[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 a = reinterpret_cast<const uint4*>(p)[i];
      pp[4 * i + 0] = a.x;
      pp[4 * i + 1] = a.y;
      pp[4 * i + 2] = a.z;
      pp[4 * i + 3] = a.w;
    }
    // four independent dot chains (one per weight dword) keep v_dot2 latency
    // off the critical path
    float t[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t u = wd[d];
      const uint32_t u8 = u >> 8;
      float a = dot2((u & 0x000F000Fu) ^ 0x64086408u, pp[4 * d + 0], 0.f);
      a = dot2((u & 0x00F000F0u) ^ 0x64806480u, pp[4 * d + 1], a);
      a = dot2((u8 & 0x000F000Fu) ^ 0x64086408u, pp[4 * d + 2], a);
      t[d] = dot2((u8 & 0x00F000F0u) ^ 0x64806480u, pp[4 * d + 3], a);
    }
    return ((t[0] + t[1]) + (t[2] + t[3])) + __builtin_bit_cast(float, p[16]);  // caller scales
  }
}

// Eight consecutive activations starting at 8*c (16- or 32-byte aligned).
template <bool XF32>
__device__ __forceinline__ void load_x8(const void* x, int c, float* v) {
  if constexpr (XF32) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4* q = reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + 8 * c);
    const f32x4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + 8 * c);
    const uint32_t d[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f16x2 h = as_h2(d[q]);
      v[2 * q] = static_cast<float>(h.x);
      v[2 * q + 1] = static_cast<float>(h.y);
    }
  }
}

template <bool XF32>
__device__ __forceinline__ float load_x(const void* x, int i) {
  if constexpr (XF32) return static_cast<const float*>(x)[i];
  else return h2f(static_cast<const uint16_t*>(x)[i]);
}

// ---------------------------------------------------------------------------
// Kernel pieces.
// ---------------------------------------------------------------------------
// One pipeline slot: kUnroll weight chunks (and their raw fp16 group scales)
// of one lane.
struct Slot {
  u32x4 w[kUnroll];
  uint32_t g[kUnroll];
};

template <int FMT>
__device__ __forceinline__ void load_slot(const GemvGeom& g, const BatchPos& bp, const uint8_t* W,
                                          const uint16_t* G, int r, int j, Slot& s) {
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    s.w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W + weight_offset(g, bp, r, j, u)));
    if constexpr (FMT == CPI_W_I4G32) s.g[u] = G[scale_index(g, bp, r, j, u)];
  }
}

template <int FMT>
__device__ __forceinline__ float compute_slot(const uint32_t* lds_lane, const GemvGeom& g,
                                              const BatchPos& bp, int j, const Slot& s, float acc) {
  using F = FmtT<FMT>;
  const uint32_t* pb = lds_lane + bp.cbase * F::kStride;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (!bp.full && bp.cbase + u * kChunkCols + j >= g.nchunks) continue;  // past the row end
    const uint32_t* pc = pb + u * kChunkCols * F::kStride;
    if constexpr (FMT == CPI_W_I4G32) acc = fmaf(h2f(static_cast<uint16_t>(s.g[u])), chunk_dot<FMT>(s.w[u], pc, 0.f), acc);
    else if constexpr (FMT == CPI_W_I4ROW) acc += chunk_dot<FMT>(s.w[u], pc, 0.f);
    else acc = chunk_dot<FMT>(s.w[u], pc, acc);
  }
  return acc;
}

struct TileCtx {
  int row;
  bool row_ok;
};

// Reduce the 8 chunk-column partials of each row and run the epilogue.
template <int FMT, int EPI>
__device__ __forceinline__ void finish_tile(const GemvParams& p, int t, int r, int j, const TileCtx& tc,
                                            float acc) {
  acc = group_sum<kChunkCols>(acc);
  const int row = tc.row;
  const bool row_ok = tc.row_ok;
  if constexpr (FMT == CPI_W_I8ROW || FMT == CPI_W_I4ROW) {
    const float* sc = static_cast<const float*>(p.scales);
    acc *= (p.scale_count == 1) ? sc[0] : sc[row_ok ? row : p.R - 1];
  }
  if constexpr (EPI == CPI_EPI_STORE_F32) {
    if (j == 0 && row_ok) static_cast<float*>(p.y)[row] = acc;
  } else if constexpr (EPI == CPI_EPI_STORE_F16) {
    if (j == 0 && row_ok) static_cast<uint16_t*>(p.y)[row] = f2h(acc);
  } else if constexpr (EPI == EPI_DUAL_F16) {
    if (j == 0 && row_ok) {
      if (row < p.rows_a) static_cast<uint16_t*>(p.y)[row] = f2h(acc);
      else static_cast<uint16_t*>(p.y2)[row - p.rows_a] = f2h(acc);
    }
  } else if constexpr (EPI == CPI_EPI_RESID_ADD) {
    if (j == 0 && row_ok) static_cast<float*>(p.y)[row] += acc;
  } else if constexpr (EPI == CPI_EPI_SWIGLU) {
    // tile t rows: [w1 4t..4t+3 | w3 4t..4t+3]; partner lane = lane ^ 32.
    const float other = __shfl_xor(acc, 32, kWave);
    if (j == 0 && r < 4) {
      const float g = acc;
      static_cast<float*>(p.y)[t * 4 + r] = (g / (1.f + expf(-g))) * other;
    }
  } else if constexpr (EPI == CPI_EPI_QKV_ROPE) {
    const float other = __shfl_xor(acc, 32, kWave);
    const int hd = p.hd;
    const int half = hd >> 1;
    const int tiles_per_head = hd / kTileRows;
    const int q_tiles = p.nh * tiles_per_head;
    const int k_tiles = p.nkv * tiles_per_head;
    const int kvdim = p.nkv * hd;
    const int pos = *p.position;
    if (j == 0) {
      if (t < q_tiles + k_tiles) {
        const bool is_q = t < q_tiles;
        const int u = is_q ? t : t - q_tiles;
        const int head = u / tiles_per_head;
        const int bb = u % tiles_per_head;
        const int dd = 4 * bb + (r & 3);
        const float c = p.rope_cos[static_cast<size_t>(pos) * half + dd];
        const float s = p.rope_sin[static_cast<size_t>(pos) * half + dd];
        float outv;
        int d;
        if (r < 4) {  // acc = x0, other = x1
          outv = acc * c - other * s;
          d = dd;
        } else {      // acc = x1, other = x0
          outv = other * s + acc * c;
          d = dd + half;
        }
        if (is_q) {
          static_cast<float*>(p.y)[head * hd + d] = outv;
        } else if (pos < p.max_ctx) {
          p.k_cache[static_cast<size_t>(pos) * kvdim + head * hd + d] = f2h(outv);
        }
      } else {
        const int vr = (t - q_tiles - k_tiles) * kTileRows + r;
        if (pos < p.max_ctx && vr < kvdim) p.v_cache[static_cast<size_t>(pos) * kvdim + vr] = f2h(acc);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel.  A workgroup's 4 waves cover TPW = 4/KS tiles per iteration, each
// tile split into KS K-segments (one wave each, equal batch counts, reduced
// through LDS in a fixed order).  Each wave walks its work as a flat sequence
// of batches through a ring of three register slots (prefetch distance two);
// the first two batches are issued before the activation prologue.
// ---------------------------------------------------------------------------
template <int FMT, int EPI, bool XF32>
__global__ void __launch_bounds__(kBlock) gemv_kernel(GemvParams p, int ks) {
  using F = FmtT<FMT>;
  extern __shared__ __align__(16) uint32_t lds[];
  __shared__ float red[kWavesPerBlock];
  __shared__ float part[kWavesPerBlock][kTileRows];

  const int K = p.K;
  const GemvGeom geo = make_geom(p.R, K, F::kElems, ks, gridDim.x);
  const int nchunks = geo.nchunks;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane / kChunkCols;
  const int j = lane % kChunkCols;
  const int tpw = geo.tpw;
  const int seg = wave % ks;
  const int tiles = geo.tiles;
  const int nbs = geo.nbs;
  const int wtile = wave / ks;
  const uint8_t* W = static_cast<const uint8_t*>(p.w);
  const uint16_t* G = static_cast<const uint16_t*>(p.scales);
  const int total = my_groups(geo, blockIdx.x) * nbs;
  auto addr_of = [&](int g, int bb) { return batch_pos(geo, blockIdx.x, wave, g, bb); };

  // ---- prologue part 1: activations (and norm weights) into registers
  constexpr int MAXC = 64 / F::kElems;  // chunks per thread held in registers
  const bool in_regs = nchunks <= MAXC * kBlock;
  float xr[MAXC][F::kElems];
  uint32_t nr[MAXC][F::kElems / 2];
  if (in_regs) {
#pragma unroll
    for (int q = 0; q < MAXC; ++q) {
      const int c = threadIdx.x + q * kBlock;
      if (c < nchunks) {
#pragma unroll
        for (int e8 = 0; e8 < F::kElems / 8; ++e8) {
          load_x8<XF32>(p.x, c * (F::kElems / 8) + e8, &xr[q][8 * e8]);
          if (p.norm_w != nullptr) {
            const u32x4 nw = *reinterpret_cast<const u32x4*>(p.norm_w + (c * (F::kElems / 8) + e8) * 8);
            nr[q][4 * e8 + 0] = nw.x; nr[q][4 * e8 + 1] = nw.y;
            nr[q][4 * e8 + 2] = nw.z; nr[q][4 * e8 + 3] = nw.w;
          }
        }
      }
    }
  }

  // ---- first two batches in flight before the activations are consumed
  int gi = blockIdx.x, b = 0;
  int g1 = gi, b1 = 1, g2, b2;
  if (b1 == nbs) { b1 = 0; g1 += gridDim.x; }
  g2 = g1; b2 = b1 + 1;
  if (b2 == nbs) { b2 = 0; g2 += gridDim.x; }
  Slot sa, sb, sc;
  BatchPos A0 = addr_of(gi, b), A1 = addr_of(g1, b1);
  if (total > 0) {
    load_slot<FMT>(geo, A0, W, G, r, j, sa);
    load_slot<FMT>(geo, A1, W, G, r, j, sb);
  }

  // ---- prologue part 2: RMSNorm statistics and activation preparation
  {
    float inv_rms = 1.f;
    if (in_regs) {
      if (p.norm_w != nullptr) {
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < MAXC; ++q)
          if (threadIdx.x + q * kBlock < nchunks)
#pragma unroll
            for (int e = 0; e < F::kElems; ++e) ss += xr[q][e] * xr[q][e];
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        lds_barrier();
        ss = 0.f;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) ss += red[w];
        inv_rms = 1.f / sqrtf(ss / static_cast<float>(K) + p.eps);
      }
#pragma unroll
      for (int q = 0; q < MAXC; ++q) {
        const int c = threadIdx.x + q * kBlock;
        if (c < nchunks) {
          if (p.norm_w != nullptr) {
#pragma unroll
            for (int e2 = 0; e2 < F::kElems / 2; ++e2) {
              const f16x2 h = as_h2(nr[q][e2]);
              xr[q][2 * e2] = (inv_rms * xr[q][2 * e2]) * static_cast<float>(h.x);
              xr[q][2 * e2 + 1] = (inv_rms * xr[q][2 * e2 + 1]) * static_cast<float>(h.y);
            }
          }
          prep_chunk<FMT>(xr[q], lds + c * F::kStride);
        }
      }
    } else {
      // large K: strided fallback (activations re-read from global)
      if (p.norm_w != nullptr) {
        float ss = 0.f;
        for (int c = threadIdx.x; c < K / 8; c += kBlock) {
          float v[8];
          load_x8<XF32>(p.x, c, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        lds_barrier();
        ss = 0.f;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) ss += red[w];
        inv_rms = 1.f / sqrtf(ss / static_cast<float>(K) + p.eps);
      }
      for (int c = threadIdx.x; c < nchunks; c += kBlock) {
        float v[F::kElems];
#pragma unroll
        for (int e8 = 0; e8 < F::kElems / 8; ++e8) {
          load_x8<XF32>(p.x, c * (F::kElems / 8) + e8, v + 8 * e8);
          if (p.norm_w != nullptr) {
            const u32x4 nw = *reinterpret_cast<const u32x4*>(p.norm_w + (c * (F::kElems / 8) + e8) * 8);
            const uint32_t nd[4] = {nw.x, nw.y, nw.z, nw.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f16x2 h = as_h2(nd[q]);
              v[8 * e8 + 2 * q] = (inv_rms * v[8 * e8 + 2 * q]) * static_cast<float>(h.x);
              v[8 * e8 + 2 * q + 1] = (inv_rms * v[8 * e8 + 2 * q + 1]) * static_cast<float>(h.y);
            }
          }
        }
        prep_chunk<FMT>(v, lds + c * F::kStride);
      }
    }
  }
  lds_barrier();

  const uint32_t* lds_lane = lds + j * F::kStride;
  float acc = 0.f;
  int done = 0;
  // One pipeline step: issue position (g2, b2) into SN, consume (gi, b) from SC.
#define CPI_GEMV_STEP(SC, SN)                                                                  \
  {                                                                                            \
    const BatchPos A2 = addr_of(g2, b2);                                                       \
    load_slot<FMT>(geo, A2, W, G, r, j, SN);                                                   \
    const int t = gi * tpw + wtile;                                                            \
    const bool tile_ok = t < tiles;                                                            \
    acc = compute_slot<FMT>(lds_lane, geo, A0, j, SC, acc);                                    \
    if (b == nbs - 1) {                                                                        \
      TileCtx tc;                                                                              \
      tc.row = t * kTileRows + r;                                                              \
      tc.row_ok = tile_ok && tc.row < p.R;                                                     \
      if (ks == 1) {                                                                           \
        if (tile_ok) finish_tile<FMT, EPI>(p, t, r, j, tc, acc);                               \
      } else {                                                                                 \
        const float v = group_sum<kChunkCols>(acc);                                            \
        if (j == 0) part[wave][r] = v;                                                         \
        lds_barrier();                                                                         \
        if (seg == 0 && tile_ok) {                                                             \
          float tot = 0.f;                                                                     \
          if (j == 0) {                                                                        \
            tot = part[wave][r];                                                               \
            for (int s2 = 1; s2 < ks; ++s2) tot += part[wave + s2][r];                         \
          }                                                                                    \
          finish_tile<FMT, EPI>(p, t, r, j, tc, tot);                                          \
        }                                                                                      \
        lds_barrier();                                                                         \
      }                                                                                        \
      acc = 0.f;                                                                               \
    }                                                                                          \
    gi = g1; b = b1; g1 = g2; b1 = b2;                                                         \
    if (++b2 == nbs) { b2 = 0; g2 += gridDim.x; }                                              \
    A0 = A1; A1 = A2;                                                                          \
    ++done;                                                                                    \
  }
  while (done < total) {  // `total` is uniform across the workgroup
    CPI_GEMV_STEP(sa, sc)
    if (done >= total) break;
    CPI_GEMV_STEP(sb, sa)
    if (done >= total) break;
    CPI_GEMV_STEP(sc, sb)
  }
#undef CPI_GEMV_STEP
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {

int g_max_blocks = 4096;
int g_force_ks = 0;

template <int FMT>
size_t lds_bytes(int K) {
  return static_cast<size_t>(K / FmtT<FMT>::kElems) * FmtT<FMT>::kStride * sizeof(uint32_t);
}

template <int FMT, int EPI, bool XF32>
hipError_t launch(const GemvParams& p_in, hipStream_t s) {
  const GemvParams& p = p_in;
  int ks = 1, blocks = 1;
  plan_launch(p.R, p.K, FmtT<FMT>::kElems, g_max_blocks, g_force_ks, &ks, &blocks);
  const size_t lds = lds_bytes<FMT>(p.K);
  hipLaunchKernelGGL((gemv_kernel<FMT, EPI, XF32>), dim3(blocks), dim3(kBlock), lds, s, p, ks);
  return hipGetLastError();
}

template <int FMT, bool XF32>
hipError_t dispatch_epi(int epi, const GemvParams& p, hipStream_t s) {
  switch (epi) {
    case CPI_EPI_STORE_F32: return launch<FMT, CPI_EPI_STORE_F32, XF32>(p, s);
    case CPI_EPI_STORE_F16: return launch<FMT, CPI_EPI_STORE_F16, XF32>(p, s);
    case CPI_EPI_RESID_ADD: return launch<FMT, CPI_EPI_RESID_ADD, XF32>(p, s);
    case CPI_EPI_SWIGLU: return launch<FMT, CPI_EPI_SWIGLU, XF32>(p, s);
    case CPI_EPI_QKV_ROPE: return launch<FMT, CPI_EPI_QKV_ROPE, XF32>(p, s);
    case EPI_DUAL_F16: return launch<FMT, EPI_DUAL_F16, XF32>(p, s);
  }
  return hipErrorInvalidValue;
}

template <int FMT>
hipError_t dispatch_x(int epi, bool xf32, const GemvParams& p, hipStream_t s) {
  return xf32 ? dispatch_epi<FMT, true>(epi, p, s) : dispatch_epi<FMT, false>(epi, p, s);
}

}  // namespace

void gemv_set_max_blocks(int n) { g_max_blocks = n > 0 ? n : 4096; }
void gemv_set_ksplit(int n) { g_force_ks = (n == 1 || n == 2 || n == 4) ? n : 0; }

hipError_t gemv_launch(int wfmt, int epi, bool xf32, const GemvParams& p, hipStream_t s) {
  static const bool env_once = [] {
    if (const char* v = getenv("CPI_GEMV_KSPLIT")) gemv_set_ksplit(atoi(v));
    if (const char* v = getenv("CPI_GEMV_MAX_BLOCKS")) gemv_set_max_blocks(atoi(v));
    return true;
  }();
  (void)env_once;
  switch (wfmt) {
    case CPI_W_F16: return dispatch_x<CPI_W_F16>(epi, xf32, p, s);
    case CPI_W_I8ROW: return dispatch_x<CPI_W_I8ROW>(epi, xf32, p, s);
    case CPI_W_I4ROW: return dispatch_x<CPI_W_I4ROW>(epi, xf32, p, s);
    case CPI_W_I4G32: return dispatch_x<CPI_W_I4G32>(epi, xf32, p, s);
  }
  return hipErrorInvalidValue;
}

int gemv_elems_per_chunk(int wfmt) {
  switch (wfmt) {
    case CPI_W_F16: return 8;
    case CPI_W_I8ROW: return 16;
    case CPI_W_I4ROW:
    case CPI_W_I4G32: return 32;
  }
  return 0;
}


}  // namespace cpi

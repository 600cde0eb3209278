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
#include "common.hpp"
#include "../../include/cpi_hip.h"

namespace cpi {

constexpr int kChunkCols = 8;                 // 16-byte chunks per row per step
constexpr int kTileRows = kWave / kChunkCols; // rows per wave tile
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;
constexpr int kUnroll = 4;

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
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      acc = dot2(wd[d], h[d], acc);
      acc = dot2(wd[d], l[d], acc);
    }
    return acc;
  } else if constexpr (FMT == CPI_W_I8ROW) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    const uint32_t pp[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float t = __builtin_bit_cast(float, p[8]);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t u = wd[d] ^ 0x80808080u;
      t = dot2((u & 0x00FF00FFu) | 0x64006400u, pp[2 * d], t);
      t = dot2(((u >> 8) & 0x00FF00FFu) | 0x64006400u, pp[2 * d + 1], t);
    }
    return acc + t;
  } else {
    uint32_t pp[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 a = reinterpret_cast<const uint4*>(p)[i];
      pp[4 * i + 0] = a.x;
      pp[4 * i + 1] = a.y;
      pp[4 * i + 2] = a.z;
      pp[4 * i + 3] = a.w;
    }
    float t = __builtin_bit_cast(float, p[16]);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t u = wd[d] ^ 0x88888888u;
      const uint32_t u8 = u >> 8;
      t = dot2((u & 0x000F000Fu) | 0x64006400u, pp[4 * d + 0], t);
      t = dot2((u & 0x00F000F0u) | 0x64006400u, pp[4 * d + 1], t);
      t = dot2((u8 & 0x000F000Fu) | 0x64006400u, pp[4 * d + 2], t);
      t = dot2((u8 & 0x00F000F0u) | 0x64006400u, pp[4 * d + 3], t);
    }
    return t;  // caller applies the group scale / accumulates
  }
}

template <bool XF32>
__device__ __forceinline__ float load_x(const void* x, int i) {
  if constexpr (XF32) return static_cast<const float*>(x)[i];
  else return h2f(static_cast<const uint16_t*>(x)[i]);
}

// ---------------------------------------------------------------------------
// Kernel.
// ---------------------------------------------------------------------------
template <int FMT, int EPI, bool XF32>
__global__ void __launch_bounds__(kBlock) gemv_kernel(GemvParams p) {
  using F = FmtT<FMT>;
  extern __shared__ __align__(16) uint32_t lds[];
  __shared__ float red[kWavesPerBlock];

  const int K = p.K;
  const int nchunks = K / F::kElems;

  // ---- prologue: optional RMSNorm statistics, then activation preparation
  float inv_rms = 1.f;
  if (p.norm_w != nullptr) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < K; i += kBlock) {
      const float v = load_x<XF32>(p.x, i);
      ss += v * v;
    }
    ss = block_sum(ss, red);
    inv_rms = 1.f / sqrtf(ss / static_cast<float>(K) + p.eps);
  }
  for (int c = threadIdx.x; c < nchunks; c += kBlock) {
    float v[F::kElems];
#pragma unroll
    for (int e = 0; e < F::kElems; ++e) {
      const int i = c * F::kElems + e;
      float xv = load_x<XF32>(p.x, i);
      if (p.norm_w != nullptr) xv = (inv_rms * xv) * h2f(p.norm_w[i]);
      v[e] = xv;
    }
    prep_chunk<FMT>(v, lds + c * F::kStride);
  }
  __syncthreads();

  // ---- main loop: one wave per 8-row tile, grid-stride over tiles
  const int lane = threadIdx.x & (kWave - 1);
  const int r = lane / kChunkCols;
  const int j = lane % kChunkCols;
  const int waves_total = gridDim.x * kWavesPerBlock;
  const int tiles = (p.R + kTileRows - 1) / kTileRows;
  const int steps = (nchunks + kChunkCols - 1) / kChunkCols;
  const size_t row_bytes = static_cast<size_t>(K) * 16 / F::kElems;

  for (int t = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave; t < tiles; t += waves_total) {
    const int row = t * kTileRows + r;
    const bool row_ok = row < p.R;
    const int rowc = row_ok ? row : (p.R - 1);
    const uint8_t* wrow = static_cast<const uint8_t*>(p.w) + static_cast<size_t>(rowc) * row_bytes;
    const uint16_t* grow = nullptr;
    if constexpr (FMT == CPI_W_I4G32)
      grow = static_cast<const uint16_t*>(p.scales) + static_cast<size_t>(rowc) * nchunks;

    float acc = 0.f;
    for (int s0 = 0; s0 < steps; s0 += kUnroll) {
      u32x4 wv[kUnroll];
      float gs[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int c = (s0 + u) * kChunkCols + j;
        if (c < nchunks) {
          wv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow) + c);
          if constexpr (FMT == CPI_W_I4G32) gs[u] = h2f(grow[c]);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int c = (s0 + u) * kChunkCols + j;
        if (c < nchunks) {
          const uint32_t* pc = lds + c * F::kStride;
          if constexpr (FMT == CPI_W_I4G32) {
            acc = fmaf(gs[u], chunk_dot<FMT>(wv[u], pc, 0.f), acc);
          } else if constexpr (FMT == CPI_W_I4ROW) {
            acc += chunk_dot<FMT>(wv[u], pc, 0.f);
          } else {
            acc = chunk_dot<FMT>(wv[u], pc, acc);
          }
        }
      }
    }
    acc = group_sum<kChunkCols>(acc);
    if constexpr (FMT == CPI_W_I8ROW || FMT == CPI_W_I4ROW) {
      const float* sc = static_cast<const float*>(p.scales);
      acc *= (p.scale_count == 1) ? sc[0] : sc[rowc];
    }

    // ---- epilogues (value of row r lives in lane r*8)
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
          const int b = u % tiles_per_head;
          const int dd = 4 * b + (r & 3);
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
          if (pos < p.max_ctx && vr < kvdim)
            p.v_cache[static_cast<size_t>(pos) * kvdim + vr] = f2h(acc);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {

int g_max_blocks = 1024;

template <int FMT>
size_t lds_bytes(int K) {
  return static_cast<size_t>(K / FmtT<FMT>::kElems) * FmtT<FMT>::kStride * sizeof(uint32_t);
}

template <int FMT, int EPI, bool XF32>
hipError_t launch(const GemvParams& p, hipStream_t s) {
  const int tiles = (p.R + kTileRows - 1) / kTileRows;
  int blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > g_max_blocks) blocks = g_max_blocks;
  const size_t lds = lds_bytes<FMT>(p.K);
  hipLaunchKernelGGL((gemv_kernel<FMT, EPI, XF32>), dim3(blocks), dim3(kBlock), lds, s, p);
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

hipError_t gemv_launch(int wfmt, int epi, bool xf32, const GemvParams& p, hipStream_t s) {
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

void gemv_set_max_blocks(int n) { g_max_blocks = n > 0 ? n : 1024; }

}  // namespace cpi

// Chunked prefill for gfx950: a dequantising GEMM on MFMA and a causal
// flash-attention over the KV cache, both for a chunk of M prompt tokens.
//
// Replaces, for the resident engine, what the reference's prefill_prompt
// (src/engine/llama_engine_generation.cpp:39-454) issues per layer: the
// cuBLASLt GEMMs of detail::dispatch_linear_rowmajor_weight
// (src/engine/llama_engine.cpp:69-249), launch_rope_inplace_batched
// (src/kernels/kernels.cu:305-343), the per-token KV copies,
// launch_attention_prefill (src/kernels/kernels.cu:435-539, 634-673),
// launch_add_inplace and launch_silu_mul.  Unlike the reference, the weights
// stay in their low-bit format: each workgroup dequantises its weight tile
// into LDS as fp16 and feeds v_mfma_f32_16x16x32_f16.
//
// Conventions shared by both kernels (16x16x32 f16 MFMA):
//   lane l, group g = l / 16, column c = l % 16
//   A operand: 8 fp16 of row c, B operand: 8 fp16 of column c, at k positions
//   that are a function of (g, j) only, identical for A and B;
//   D (4 fp32): rows 4 g + r (r = 0..3), column c.
#include "common.hpp"
#include "../../include/cpi_hip.h"

namespace cpi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// RMSNorm of fp32 rows into fp16 rows: y = fp16((x * inv_rms) * w), fp32
// statistics (kernels.cu:36-99 semantics, cpu_engine.cpp:392-405 order).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) rmsnorm_rows_kernel(const float* x, const uint16_t* w, uint16_t* y,
                                                           int cols, float eps) {
  __shared__ float red[4];
  const float* xr = x + static_cast<size_t>(blockIdx.x) * cols;
  uint16_t* yr = y + static_cast<size_t>(blockIdx.x) * cols;
  float ss = 0.f;
  for (int i = threadIdx.x; i < cols; i += 256) ss += xr[i] * xr[i];
  ss = block_sum(ss, red);
  const float inv = 1.f / sqrtf(ss / static_cast<float>(cols) + eps);
  for (int i = threadIdx.x; i < cols; i += 256) yr[i] = f2h((inv * xr[i]) * h2f(w[i]));
}

// ---------------------------------------------------------------------------
// GEMM  Y[m, n] = sum_k X[m, k] W[n, k]  (W row-major [N, K] in a CPI_W_*
// format, X fp16 [M, K]) with the engine's fused epilogues.
// Tile: 64 weight rows x 64 tokens x 64 k per step, 4 waves, each wave 32 rows
// x 32 tokens (2 x 2 MFMA blocks).  Weight and activation tiles are staged in
// LDS (double buffered) with an 8-half row pad; global loads of step s+1 are
// in flight while step s runs on the matrix cores.
// ---------------------------------------------------------------------------
struct PGemmParams {
  const uint8_t* w;
  const void* scales;
  int scale_count;
  int N, K, M;
  const uint16_t* x;
  int epi;
  void* y;
  int nh, nkv, hd;
  int start;
  const float* rope_cos;
  const float* rope_sin;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int max_ctx;
};

constexpr int kPT = 64;        // tile rows / tokens / k
constexpr int kPLd = kPT + 8;  // LDS row stride in halves (bank spread)

// Weight bytes of 16 consecutive k values of one row.
template <int FMT> struct PW;
template <> struct PW<CPI_W_F16> { typedef u32x4 T[2]; static constexpr int kBytes = 32; };
template <> struct PW<CPI_W_I8ROW> { typedef u32x4 T[1]; static constexpr int kBytes = 16; };
template <> struct PW<CPI_W_I4ROW> { typedef uint2 T[1]; static constexpr int kBytes = 8; };
template <> struct PW<CPI_W_I4G32> : PW<CPI_W_I4ROW> {};

// Offset-binary bytes (b' = q + 128) or nibbles (n' = q + 8) sit under the
// exponent of 1024.0 as fp16; subtracting the bias gives q exactly.
__device__ __forceinline__ uint32_t pair_bits(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel) | 0x64006400u;
}

// 16 fp16 weights (q, or q * group scale for I4G32) in natural k order.
template <int FMT>
__device__ __forceinline__ void dequant16(const typename PW<FMT>::T& raw, uint16_t gscale, uint32_t* out) {
  if constexpr (FMT == CPI_W_F16) {
    out[0] = raw[0].x; out[1] = raw[0].y; out[2] = raw[0].z; out[3] = raw[0].w;
    out[4] = raw[1].x; out[5] = raw[1].y; out[6] = raw[1].z; out[7] = raw[1].w;
  } else if constexpr (FMT == CPI_W_I8ROW) {
    const uint32_t d[4] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w};
    const f16x2 bias = {static_cast<f16>(-1152.f), static_cast<f16>(-1152.f)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = d[i] ^ 0x80808080u;
      const f16x2 a = as_h2(pair_bits(0u, v, 0x0c010c00u)) + bias;
      const f16x2 b = as_h2(pair_bits(0u, v, 0x0c030c02u)) + bias;
      out[2 * i] = __builtin_bit_cast(uint32_t, a);
      out[2 * i + 1] = __builtin_bit_cast(uint32_t, b);
    }
  } else {
    const uint32_t d[2] = {raw[0].x, raw[0].y};
    const f16x2 bias = {static_cast<f16>(-1032.f), static_cast<f16>(-1032.f)};
    f16x2 sc;
    if constexpr (FMT == CPI_W_I4G32) {
      sc.x = __builtin_bit_cast(f16, gscale);
      sc.y = sc.x;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t v = d[i] ^ 0x88888888u;
      const uint32_t lo = v & 0x0F0F0F0Fu;         // even k of each byte
      const uint32_t hi = (v >> 4) & 0x0F0F0F0Fu;  // odd k
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t sel = 0x0c000c00u | (static_cast<uint32_t>(b + 4) << 16) | static_cast<uint32_t>(b);
        f16x2 q = as_h2(pair_bits(hi, lo, sel)) + bias;
        if constexpr (FMT == CPI_W_I4G32) q = q * sc;
        out[4 * i + b] = __builtin_bit_cast(uint32_t, q);
      }
    }
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.f + expf(-g)); }

template <int FMT>
__global__ void __launch_bounds__(256) pgemm_kernel(PGemmParams p) {
  __shared__ __align__(16) uint16_t Ws[2][kPT * kPLd];
  __shared__ __align__(16) uint16_t Xs[2][kPT * kPLd];
  __shared__ float Cs[kPT][kPT + 1];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int n0 = blockIdx.x * kPT;
  const int m0 = blockIdx.y * kPT;
  const int K = p.K;

  // loader role: row / token t/4, 16 k values at 16*(t%4)
  const int lr = t >> 2, lq = t & 3;
  const int wrow = min(n0 + lr, p.N - 1);
  const int xtok = min(m0 + lr, p.M - 1);
  const size_t row_bytes = FMT == CPI_W_F16 ? 2u * K : (FMT == CPI_W_I8ROW ? static_cast<size_t>(K) : K / 2u);
  const uint8_t* wsrc = p.w + static_cast<size_t>(wrow) * row_bytes + lq * PW<FMT>::kBytes;
  const uint16_t* xsrc = p.x + static_cast<size_t>(xtok) * K + 16 * lq;
  const uint16_t* gsrc = FMT == CPI_W_I4G32
                             ? static_cast<const uint16_t*>(p.scales) + static_cast<size_t>(wrow) * (K / 32) + lq / 2
                             : nullptr;

  typename PW<FMT>::T wr;
  u32x4 xr[2];
  uint16_t gs = 0;
  auto load = [&](int kt) {
    const uint8_t* ws = wsrc + static_cast<size_t>(kt) * (PW<FMT>::kBytes * 4);
    if constexpr (FMT == CPI_W_F16) {
      wr[0] = *reinterpret_cast<const u32x4*>(ws);
      wr[1] = *reinterpret_cast<const u32x4*>(ws + 16);
    } else if constexpr (FMT == CPI_W_I8ROW) {
      wr[0] = *reinterpret_cast<const u32x4*>(ws);
    } else {
      wr[0] = *reinterpret_cast<const uint2*>(ws);
    }
    if constexpr (FMT == CPI_W_I4G32) gs = gsrc[kt * 2];
    const uint16_t* xs = xsrc + static_cast<size_t>(kt) * kPT;
    xr[0] = *reinterpret_cast<const u32x4*>(xs);
    xr[1] = *reinterpret_cast<const u32x4*>(xs + 8);
  };
  auto stage = [&](int buf) {
    uint32_t d[8];
    dequant16<FMT>(wr, gs, d);
    u32x4* wdst = reinterpret_cast<u32x4*>(&Ws[buf][lr * kPLd + 16 * lq]);
    wdst[0] = u32x4{d[0], d[1], d[2], d[3]};
    wdst[1] = u32x4{d[4], d[5], d[6], d[7]};
    u32x4* xdst = reinterpret_cast<u32x4*>(&Xs[buf][lr * kPLd + 16 * lq]);
    xdst[0] = xr[0];
    xdst[1] = xr[1];
  };

  // wave tile: rows 32*(wave/2), tokens 32*(wave%2)
  const int wr0 = 32 * (wave >> 1), wt0 = 32 * (wave & 1);
  f4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int nk = K / kPT;
  load(0);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    stage(buf);
    __syncthreads();
    if (kt + 1 < nk) load(kt + 1);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      h8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const h8*>(&Ws[buf][(wr0 + 16 * i + c) * kPLd + 32 * s + 8 * g]);
        b[i] = *reinterpret_cast<const h8*>(&Xs[buf][(wt0 + 16 * i + c) * kPLd + 32 * s + 8 * g]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
    }
  }

  // D rows are weight rows (n), columns tokens (m)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) Cs[wr0 + 16 * i + 4 * g + r][wt0 + 16 * j + c] = acc[i][j][r];
  __syncthreads();

  const float* rsc = (FMT == CPI_W_I8ROW || FMT == CPI_W_I4ROW) ? static_cast<const float*>(p.scales) : nullptr;
  for (int e = t; e < kPT * kPT; e += 256) {
    const int nl = e & (kPT - 1), ml = e / kPT;
    const int n = n0 + nl, m = m0 + ml;
    if (n >= p.N || m >= p.M) continue;
    auto val = [&](int nll) {
      float v = Cs[nll][ml];
      if (rsc) v *= p.scale_count == 1 ? rsc[0] : rsc[n0 + nll];
      return v;
    };
    const float v = val(nl);
    switch (p.epi) {
      case CPI_EPI_STORE_F32: static_cast<float*>(p.y)[static_cast<size_t>(m) * p.N + n] = v; break;
      case CPI_EPI_STORE_F16: static_cast<uint16_t*>(p.y)[static_cast<size_t>(m) * p.N + n] = f2h(v); break;
      case CPI_EPI_RESID_ADD: static_cast<float*>(p.y)[static_cast<size_t>(m) * p.N + n] += v; break;
      case CPI_EPI_SWIGLU: {
        // tile of 8 rows: w1 rows 4T..4T+3, then the matching w3 rows
        const int r = n & 7;
        if (r < 4) {
          const float u = val(nl + 4);
          static_cast<uint16_t*>(p.y)[static_cast<size_t>(m) * (p.N / 2) + (n >> 3) * 4 + r] = f2h(silu(v) * u);
        }
        break;
      }
      case CPI_EPI_QKV_ROPE: {
        const int T = n >> 3, r = n & 7;
        const int hd = p.hd, half = hd >> 1, tph = hd / 8;
        const int q_tiles = p.nh * tph, k_tiles = p.nkv * tph;
        const int kvdim = p.nkv * hd;
        const int pos = p.start + m;
        if (T < q_tiles + k_tiles) {
          const bool is_q = T < q_tiles;
          const int u = is_q ? T : T - q_tiles;
          const int head = u / tph;
          const int dd = 4 * (u % tph) + (r & 3);
          const float other = val(nl ^ 4);
          const float cs = p.rope_cos[static_cast<size_t>(pos) * half + dd];
          const float sn = p.rope_sin[static_cast<size_t>(pos) * half + dd];
          float outv;
          int d;
          if (r < 4) {
            outv = v * cs - other * sn;
            d = dd;
          } else {
            outv = other * sn + v * cs;
            d = dd + half;
          }
          if (is_q)
            static_cast<uint16_t*>(p.y)[static_cast<size_t>(m) * p.nh * hd + head * hd + d] = f2h(outv);
          else if (pos < p.max_ctx)
            p.k_cache[static_cast<size_t>(pos) * kvdim + head * hd + d] = f2h(outv);
        } else {
          const int vr = (T - q_tiles - k_tiles) * 8 + r;
          if (pos < p.max_ctx && vr < kvdim) p.v_cache[static_cast<size_t>(pos) * kvdim + vr] = f2h(v);
        }
        break;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Causal prefill attention.  Workgroup = (query head, 64 queries); wave w owns
// queries 16w..16w+15 of the tile.  Per 32-key step the K tile [32][hd] and
// the transposed V tile [hd][32] are staged in LDS, then per wave
//   S^T = K Q^T   (D rows = keys 4g+r of the two 16-key halves, column = query)
//   online softmax per query column (fp32, base 2)
//   O^T += V^T P^T  with the key order (g, j) -> j < 4 ? 4g+j : 16+4g+(j-4),
// which is exactly the key set each lane holds after S^T: P never moves.
// Query t of the chunk sits at cache position start + t and sees keys
// (start + t - window, start + t] (all earlier keys when window <= 0),
// matching the decode attention of the same position.
// ---------------------------------------------------------------------------
struct APParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  int M, start, nh, nkv, window;
  float scale_log2;
};

template <int HD>
__global__ void __launch_bounds__(256) attn_prefill_kernel(APParams p) {
  constexpr int KLd = HD + 8;  // K tile row stride (halves)
  constexpr int VLd = 32 + 8;  // V^T tile row stride (halves)
  __shared__ __align__(16) uint16_t Ks[32 * KLd];
  __shared__ __align__(16) uint16_t Vt[HD * VLd];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int h = blockIdx.x;
  const int kvh = h / (p.nh / p.nkv);
  const int kvdim = p.nkv * HD;
  const int qdim = p.nh * HD;
  const int tile0 = blockIdx.y * 64;

  const int qi = tile0 + 16 * wave + c;  // this lane's query (column c)
  const bool qvalid = qi < p.M;
  const int qm = min(qi, p.M - 1);
  const int qpos = p.start + qm;
  const int qlo = p.window > 0 ? qpos - p.window + 1 : 0;  // first visible key

  h8 qf[HD / 32];
#pragma unroll
  for (int s = 0; s < HD / 32; ++s)
    qf[s] = *reinterpret_cast<const h8*>(p.q + static_cast<size_t>(qm) * qdim + h * HD + 32 * s + 8 * g);

  // key range of the whole tile
  const int last_q = min(tile0 + 63, p.M - 1);
  const int kend = p.start + last_q + 1;  // exclusive
  int kbeg = 0;
  if (p.window > 0) kbeg = max(0, p.start + tile0 - p.window + 1);
  kbeg &= ~31;

  f4 o[HD / 16];
#pragma unroll
  for (int d = 0; d < HD / 16; ++d) o[d] = f4{0.f, 0.f, 0.f, 0.f};
  float mrun = -__builtin_inff(), lrun = 0.f;

  const uint16_t* kb = p.k + kvh * HD;
  const uint16_t* vb = p.v + kvh * HD;
  for (int kt = kbeg; kt < kend; kt += 32) {
    __syncthreads();  // previous step's readers are done with the tiles
    // K tile: 32 keys x HD, 16-byte pieces
    for (int u = t; u < 32 * (HD / 8); u += 256) {
      const int key = u / (HD / 8), piece = u % (HD / 8);
      const int kp = min(kt + key, kend - 1);
      *reinterpret_cast<u32x4*>(&Ks[key * KLd + 8 * piece]) =
          *reinterpret_cast<const u32x4*>(kb + static_cast<size_t>(kp) * kvdim + 8 * piece);
    }
    // V^T tile: units of (2 keys, 8 dims)
    for (int u = t; u < 16 * (HD / 8); u += 256) {
      const int kpair = u / (HD / 8), piece = u % (HD / 8);
      const int kp0 = min(kt + 2 * kpair, kend - 1), kp1 = min(kt + 2 * kpair + 1, kend - 1);
      const u32x4 a = *reinterpret_cast<const u32x4*>(vb + static_cast<size_t>(kp0) * kvdim + 8 * piece);
      const u32x4 b = *reinterpret_cast<const u32x4*>(vb + static_cast<size_t>(kp1) * kvdim + 8 * piece);
      const uint32_t ad[4] = {a.x, a.y, a.z, a.w}, bd[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // dims 8*piece + 2i (low halves) and + 2i + 1 (high halves)
        *reinterpret_cast<uint32_t*>(&Vt[(8 * piece + 2 * i) * VLd + 2 * kpair]) =
            __builtin_amdgcn_perm(bd[i], ad[i], 0x05040100u);
        *reinterpret_cast<uint32_t*>(&Vt[(8 * piece + 2 * i + 1) * VLd + 2 * kpair]) =
            __builtin_amdgcn_perm(bd[i], ad[i], 0x07060302u);
      }
    }
    __syncthreads();

    // S^T for keys kt + [0,16) and kt + [16,32)
    f4 sb[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      sb[b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < HD / 32; ++s) {
        const h8 ka = *reinterpret_cast<const h8*>(&Ks[(16 * b + c) * KLd + 32 * s + 8 * g]);
        sb[b] = mfma16(ka, qf[s], sb[b]);
      }
    }
    float x[8];
    float mt = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
      const int kp = kt + key;
      const bool ok = kp <= qpos && kp >= qlo;
      x[j] = ok ? sb[j >> 2][j & 3] * p.scale_log2 : -__builtin_inff();
      mt = fmaxf(mt, x[j]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mnew = fmaxf(mrun, mt);
    const bool live = mnew != -__builtin_inff();
    const float alpha = live ? exp2f(mrun - mnew) : 1.f;
    float ps = 0.f;
    h8 pf;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float e = live ? exp2f(x[j] - mnew) : 0.f;
      ps += e;
      pf[j] = static_cast<f16>(e);
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    lrun = lrun * alpha + ps;
    mrun = mnew;
#pragma unroll
    for (int d = 0; d < HD / 16; ++d) {
      const uint2 v0 = *reinterpret_cast<const uint2*>(&Vt[(16 * d + c) * VLd + 4 * g]);
      const uint2 v1 = *reinterpret_cast<const uint2*>(&Vt[(16 * d + c) * VLd + 16 + 4 * g]);
      const u32x4 vv = {v0.x, v0.y, v1.x, v1.y};
      o[d] = o[d] * alpha;
      o[d] = mfma16(__builtin_bit_cast(h8, vv), pf, o[d]);
    }
  }

  if (qvalid) {
    const float inv = 1.f / lrun;
    uint16_t* dst = p.out + static_cast<size_t>(qi) * qdim + h * HD;
#pragma unroll
    for (int d = 0; d < HD / 16; ++d)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[16 * d + 4 * g + r] = f2h(o[d][r] * inv);
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
hipError_t rmsnorm_rows_launch(const float* x, const uint16_t* w, uint16_t* y, int rows, int cols, float eps,
                               hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, s, x, w, y, cols, eps);
  return hipGetLastError();
}

hipError_t pgemm_launch(int wfmt, const PGemmParams& p, hipStream_t s) {
  const dim3 grid((p.N + kPT - 1) / kPT, (p.M + kPT - 1) / kPT);
  switch (wfmt) {
    case CPI_W_F16: hipLaunchKernelGGL(pgemm_kernel<CPI_W_F16>, grid, dim3(256), 0, s, p); break;
    case CPI_W_I8ROW: hipLaunchKernelGGL(pgemm_kernel<CPI_W_I8ROW>, grid, dim3(256), 0, s, p); break;
    case CPI_W_I4ROW: hipLaunchKernelGGL(pgemm_kernel<CPI_W_I4ROW>, grid, dim3(256), 0, s, p); break;
    case CPI_W_I4G32: hipLaunchKernelGGL(pgemm_kernel<CPI_W_I4G32>, grid, dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t attn_prefill_launch(const APParams& p, int hd, hipStream_t s) {
  const dim3 grid(p.nh, (p.M + 63) / 64);
  if (hd == 128) hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, dim3(256), 0, s, p);
  else if (hd == 64) hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, dim3(256), 0, s, p);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace cpi

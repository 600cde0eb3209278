// Decode attention for gfx950: exact online softmax, split-K over context,
// one workgroup per (KV head, context split) serving all query heads of the
// GQA group, followed by a log-sum-exp merge.
//
// Replaces src/kernels/kernels_attention_decode.cu:194-446 (tiled),
// :448-811 (chunk_stats + chunk_reduce, chunk = 32 tokens) and :868-1035
// (gqa_decode_kernel, one block per KV head and no split).  The math is the
// reference CPU attention (src/engine/cpu_engine.cpp:451-523): scores
// q.k * 1/sqrt(head_dim), softmax over [start, seq), weighted sum of V.
//
// MI355X layout choices: each K/V row of one head (head_dim fp16) is read by
// head_dim/8 lanes with 128-bit loads; K and V are read exactly once per
// workgroup and shared by the G query heads of the group; the number of
// splits is fixed per launch (graph friendly) and the split length adapts to
// the live sequence length read from device memory.
#include "common.hpp"
#include "../../include/cpi_hip.h"

namespace cpi {

constexpr int kAttnBlock = 256;
constexpr int kAttnWaves = kAttnBlock / kWave;
constexpr int kSubTile = 64;  // tokens per online-softmax step

struct AttnParams {
  const void* q;
  const uint16_t* k;
  const uint16_t* v;
  void* out;
  int seq_len;          // used when position == nullptr
  const int* position;  // seq = *position + 1
  int nh, nkv, max_ctx, window;
  int nsplit;
  float scale;
  float* scratch;       // [nh][MAXS][2] m,l  then [nh][MAXS][hd] o
};

__device__ __forceinline__ void attn_range(const AttnParams& p, int split, int& t0, int& t1,
                                           int& active) {
  int seq = p.position ? (*p.position + 1) : p.seq_len;
  if (seq > p.max_ctx) seq = p.max_ctx;
  const int start = (p.window > 0 && seq > p.window) ? seq - p.window : 0;
  const int len = seq - start;
  int chunk = (len + p.nsplit - 1) / p.nsplit;
  chunk = ((chunk + 15) / 16) * 16;
  if (chunk < 16) chunk = 16;
  active = (len + chunk - 1) / chunk;
  t0 = start + split * chunk;
  t1 = t0 + chunk;
  if (t1 > seq) t1 = seq;
}

template <int HD, int G, bool QF32>
__global__ void __launch_bounds__(kAttnBlock) attn_partial_kernel(AttnParams p) {
  constexpr int LPK = HD / 8;                 // lanes per key row (16 B each)
  constexpr int KPP = kAttnBlock / LPK;       // keys per pass
  constexpr int CB = HD / 8;                  // 16-byte column blocks of V
  constexpr int TSUB = kAttnBlock / CB;       // token subsets in the V phase
  constexpr int TSUB_W = kWave / CB;          // token subsets inside one wave
  static_assert(kSubTile % KPP == 0 || KPP % kSubTile == 0, "tile");

  __shared__ float q_s[G][HD];
  __shared__ float s_s[G][kSubTile];
  __shared__ float alpha_s[G];
  __shared__ float red_s[kAttnWaves][G][HD];

  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  int t0, t1, active;
  attn_range(p, split, t0, t1, active);
  if (split >= active) return;  // uniform per block

  const int kvdim = p.nkv * HD;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  for (int i = tid; i < G * HD; i += kAttnBlock) {
    const int g = i / HD, d = i % HD;
    const int qi = (kvh * G + g) * HD + d;
    q_s[g][d] = QF32 ? static_cast<const float*>(p.q)[qi]
                     : h2f(static_cast<const uint16_t*>(p.q)[qi]);
  }
  __syncthreads();

  // Running softmax state (m, l) per head lives in shared memory and is
  // owned by the wave that handles that head in the softmax step.
  __shared__ float m_s[G], l_s[G];
  if (tid < G) { m_s[tid] = -INFINITY; l_s[tid] = 0.f; }
  // V accumulators: this thread owns column block cb and token subset ts.
  const int cb = tid % CB;
  const int ts = tid / CB;
  float o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  __syncthreads();

  for (int base = t0; base < t1; base += kSubTile) {
    const int n = min(kSubTile, t1 - base);
    // ---- scores for up to 64 tokens
    const int kpart = tid % LPK;
    for (int kk = tid / LPK; kk < kSubTile; kk += KPP) {
      float dots[G];
#pragma unroll
      for (int g = 0; g < G; ++g) dots[g] = 0.f;
      if (kk < n) {
        const uint4 kw = *reinterpret_cast<const uint4*>(
            p.k + static_cast<size_t>(base + kk) * kvdim + kvh * HD + kpart * 8);
        const uint32_t kd[4] = {kw.x, kw.y, kw.z, kw.w};
        float kf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 h = as_h2(kd[e]);
          kf[2 * e] = static_cast<float>(h.x);
          kf[2 * e + 1] = static_cast<float>(h.y);
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < 8; ++e) dots[g] = fmaf(q_s[g][kpart * 8 + e], kf[e], dots[g]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = group_sum<LPK>(dots[g]);
        if (kpart == 0) s_s[g][kk] = (kk < n) ? d * p.scale : -INFINITY;
      }
    }
    __syncthreads();
    // ---- online softmax update: wave w handles heads w, w+4, ...
    for (int g = wave; g < G; g += kAttnWaves) {
      const float sv = s_s[g][lane];
      const float m_old = m_s[g];
      const float m_new = fmaxf(m_old, wave_max(sv));
      const float pv = (lane < n) ? expf(sv - m_new) : 0.f;
      const float psum = wave_sum(pv);
      s_s[g][lane] = pv;
      if (lane == 0) {
        const float a = expf(m_old - m_new);  // 0 on the first tile
        alpha_s[g] = a;
        l_s[g] = l_s[g] * a + psum;
        m_s[g] = m_new;
      }
    }
    __syncthreads();
    // ---- rescale and accumulate V
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float a = alpha_s[g];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= a;
    }
    for (int tt = ts; tt < n; tt += TSUB) {
      const uint4 vw = *reinterpret_cast<const uint4*>(
          p.v + static_cast<size_t>(base + tt) * kvdim + kvh * HD + cb * 8);
      const uint32_t vd[4] = {vw.x, vw.y, vw.z, vw.w};
      float vf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 h = as_h2(vd[e]);
        vf[2 * e] = static_cast<float>(h.x);
        vf[2 * e + 1] = static_cast<float>(h.y);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pw = s_s[g][tt];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pw, vf[e], o[g][e]);
      }
    }
    __syncthreads();  // s_s / alpha_s are rewritten by the next tile
  }

  // ---- reduce the token subsets: inside the wave, then across waves
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = o[g][e];
#pragma unroll
      for (int m = CB; m < kWave; m <<= 1) v += __shfl_xor(v, m, kWave);
      o[g][e] = v;
    }
  if (lane < CB) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) red_s[wave][g][cb * 8 + e] = o[g][e];
  }
  __syncthreads();
  const size_t maxs = CPI_ATTN_MAX_SPLITS;
  float* ml = p.scratch;
  float* os = p.scratch + static_cast<size_t>(p.nh) * maxs * 2;
  for (int i = tid; i < G * HD; i += kAttnBlock) {
    const int g = i / HD, d = i % HD;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) v += red_s[w][g][d];
    const int h = kvh * G + g;
    os[(static_cast<size_t>(h) * maxs + split) * HD + d] = v;
  }
  if (tid < G) {
    const int h = kvh * G + tid;
    ml[(static_cast<size_t>(h) * maxs + split) * 2 + 0] = m_s[tid];
    ml[(static_cast<size_t>(h) * maxs + split) * 2 + 1] = l_s[tid];
  }
}

// Merge the split partials of one query head:  M = max m_s,
// L = sum l_s e^(m_s - M),  out = sum o_s e^(m_s - M) / L   (fixed order).
template <int HD, bool OF32>
__global__ void __launch_bounds__(HD) attn_merge_kernel(AttnParams p) {
  const int h = blockIdx.x;
  const int d = threadIdx.x;
  int t0, t1, active;
  attn_range(p, 0, t0, t1, active);
  const size_t maxs = CPI_ATTN_MAX_SPLITS;
  const float* ml = p.scratch + static_cast<size_t>(h) * maxs * 2;
  const float* os = p.scratch + static_cast<size_t>(p.nh) * maxs * 2 + static_cast<size_t>(h) * maxs * HD;
  float M = -INFINITY;
  for (int s = 0; s < active; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.f, acc = 0.f;
  for (int s = 0; s < active; ++s) {
    const float w = expf(ml[2 * s] - M);
    L = fmaf(ml[2 * s + 1], w, L);
    acc = fmaf(os[static_cast<size_t>(s) * HD + d], w, acc);
  }
  const float r = (active > 0) ? acc / L : 0.f;
  if (OF32) static_cast<float*>(p.out)[h * HD + d] = r;
  else static_cast<uint16_t*>(p.out)[h * HD + d] = f2h(r);
}

namespace {

template <int HD, int G>
hipError_t launch_g(const AttnParams& p, bool qf32, bool of32, hipStream_t s) {
  dim3 grid(p.nkv, p.nsplit);
  if (qf32) hipLaunchKernelGGL((attn_partial_kernel<HD, G, true>), grid, dim3(kAttnBlock), 0, s, p);
  else hipLaunchKernelGGL((attn_partial_kernel<HD, G, false>), grid, dim3(kAttnBlock), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (of32) hipLaunchKernelGGL((attn_merge_kernel<HD, true>), dim3(p.nh), dim3(HD), 0, s, p);
  else hipLaunchKernelGGL((attn_merge_kernel<HD, false>), dim3(p.nh), dim3(HD), 0, s, p);
  return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const AttnParams& p, int G, bool qf32, bool of32, hipStream_t s) {
  switch (G) {
    case 1: return launch_g<HD, 1>(p, qf32, of32, s);
    case 2: return launch_g<HD, 2>(p, qf32, of32, s);
    case 4: return launch_g<HD, 4>(p, qf32, of32, s);
    case 8: return launch_g<HD, 8>(p, qf32, of32, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Split count: enough workgroups to cover the 256 CUs several times at long
// context, bounded by the scratch capacity.
int attn_num_splits(int nkv) {
  int n = 1024 / (nkv > 0 ? nkv : 1);
  if (n < 1) n = 1;
  if (n > CPI_ATTN_MAX_SPLITS) n = CPI_ATTN_MAX_SPLITS;
  return n;
}

bool attn_supported(int nh, int nkv, int hd) {
  if (nkv <= 0 || nh % nkv != 0) return false;
  const int G = nh / nkv;
  return (hd == 64 || hd == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
}

hipError_t attn_launch(const void* q, bool qf32, const uint16_t* k, const uint16_t* v, void* out,
                       bool of32, int seq_len, const int* position, int nh, int nkv, int hd,
                       int max_ctx, int window, float* scratch, hipStream_t s) {
  AttnParams p{};
  p.q = q; p.k = k; p.v = v; p.out = out;
  p.seq_len = seq_len; p.position = position;
  p.nh = nh; p.nkv = nkv; p.max_ctx = max_ctx; p.window = window;
  p.nsplit = attn_num_splits(nkv);
  p.scale = 1.f / sqrtf(static_cast<float>(hd));
  p.scratch = scratch;
  const int G = nh / nkv;
  if (hd == 64) return launch_hd<64>(p, G, qf32, of32, s);
  if (hd == 128) return launch_hd<128>(p, G, qf32, of32, s);
  return hipErrorInvalidValue;
}

}  // namespace cpi

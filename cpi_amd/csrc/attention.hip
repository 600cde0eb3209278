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

// Scratch layout (floats): [0, 64) reserved, then m,l [nh][MAXS][2], then
// o [nh][MAXS][hd].
constexpr int kCounterSlots = 64;

__device__ __forceinline__ float safe_exp_diff(float a, float m) {
  return (a == -INFINITY) ? 0.f : expf(a - m);
}

template <int HD, int G, bool QF32, bool OF32>
__global__ void __launch_bounds__(kAttnBlock) attn_kernel(AttnParams p) {
  constexpr int LPK = HD / 8;               // lanes per K/V row: 16 B each
  constexpr int NG = kAttnBlock / LPK;      // token groups per workgroup
  constexpr int GPW = kWave / LPK;          // token groups per wave
  constexpr int TB = 2;                     // tokens per group per iteration
  constexpr int CT = NG * TB;               // tokens per workgroup iteration

  __shared__ float wm[kAttnWaves][G], wl[kAttnWaves][G];
  __shared__ float wo[kAttnWaves][G][HD];
  
  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  int seq = p.position ? (*p.position + 1) : p.seq_len;
  if (seq > p.max_ctx) seq = p.max_ctx;
  const int start = (p.window > 0 && seq > p.window) ? seq - p.window : 0;
  const int len = seq - start;
  int chunk = (len + p.nsplit - 1) / p.nsplit;
  chunk = ((chunk + CT - 1) / CT) * CT;
  if (chunk < CT) chunk = CT;
  const int active = (len + chunk - 1) / chunk;
  if (split >= active) return;  // uniform per workgroup
  const int t0 = start + split * chunk;
  const int t1 = min(t0 + chunk, seq);

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int cb = tid % LPK;
  const int gid = tid / LPK;
  const int kvdim = p.nkv * HD;
  const size_t col = static_cast<size_t>(kvh) * HD + cb * 8;

  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int qi = (kvh * G + g) * HD + cb * 8 + e;
      const float v = QF32 ? static_cast<const float*>(p.q)[qi] : h2f(static_cast<const uint16_t*>(p.q)[qi]);
      qv[g][e] = v * p.scale;
    }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }

  for (int base = t0 + gid * TB; base < t1; base += CT) {
    float kf[TB][8], vf[TB][8];
    bool valid[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int t = base + tb;
      valid[tb] = t < t1;
      const size_t row = static_cast<size_t>(valid[tb] ? t : t1 - 1) * kvdim + col;
      const u32x4 kw = *reinterpret_cast<const u32x4*>(p.k + row);
      const u32x4 vw = *reinterpret_cast<const u32x4*>(p.v + row);
      const uint32_t kd[4] = {kw.x, kw.y, kw.z, kw.w};
      const uint32_t vd[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2 kh = as_h2(kd[e]);
        const f16x2 vh = as_h2(vd[e]);
        kf[tb][2 * e] = static_cast<float>(kh.x);
        kf[tb][2 * e + 1] = static_cast<float>(kh.y);
        vf[tb][2 * e] = static_cast<float>(vh.x);
        vf[tb][2 * e + 1] = static_cast<float>(vh.y);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float sc[TB];
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qv[g][e], kf[tb][e], d);
        d = group_sum<LPK>(d);
        sc[tb] = valid[tb] ? d : -INFINITY;
      }
      float mx = sc[0];
#pragma unroll
      for (int tb = 1; tb < TB; ++tb) mx = fmaxf(mx, sc[tb]);
      const float m_new = fmaxf(m[g], mx);
      if (m_new == -INFINITY) continue;  // no token seen yet by this group
      const float a = safe_exp_diff(m[g], m_new);
      float pw[TB];
      float ps = 0.f;
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        pw[tb] = safe_exp_diff(sc[tb], m_new);
        ps += pw[tb];
      }
      l[g] = l[g] * a + ps;
      m[g] = m_new;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = o[g][e] * a;
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc = fmaf(pw[tb], vf[tb][e], acc);
        o[g][e] = acc;
      }
    }
  }

  // ---- merge the token groups of this wave (shuffles over the group bits)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = m[g];
#pragma unroll
    for (int off = LPK; off < kWave; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, kWave));
    const float sc = (M == -INFINITY) ? 0.f : safe_exp_diff(m[g], M);
    float lv = l[g] * sc;
#pragma unroll
    for (int off = LPK; off < kWave; off <<= 1) lv += __shfl_xor(lv, off, kWave);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = o[g][e] * sc;
#pragma unroll
      for (int off = LPK; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
      o[g][e] = v;
    }
    if (lane < LPK) {
#pragma unroll
      for (int e = 0; e < 8; ++e) wo[wave][g][cb * 8 + e] = o[g][e];
      if (lane == 0) {
        wm[wave][g] = M;
        wl[wave][g] = lv;
      }
    }
  }
  (void)GPW;
  __syncthreads();

  // ---- merge the waves; either finish (single split) or publish a partial
  const size_t maxs = CPI_ATTN_MAX_SPLITS;
  float* ml = p.scratch + kCounterSlots;
  float* os = ml + static_cast<size_t>(p.nh) * maxs * 2;
  for (int i = tid; i < G * HD; i += kAttnBlock) {
    const int g = i / HD, d = i % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, wm[w][g]);
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float sc = safe_exp_diff(wm[w][g], M);
      L = fmaf(wl[w][g], sc, L);
      acc = fmaf(wo[w][g][d], sc, acc);
    }
    const int h = kvh * G + g;
    if (active == 1) {
      const float r = acc / L;
      if (OF32) static_cast<float*>(p.out)[h * HD + d] = r;
      else static_cast<uint16_t*>(p.out)[h * HD + d] = f2h(r);
    } else {
      os[(static_cast<size_t>(h) * maxs + split) * HD + d] = acc;
      if (d == 0) {
        ml[(static_cast<size_t>(h) * maxs + split) * 2 + 0] = M;
        ml[(static_cast<size_t>(h) * maxs + split) * 2 + 1] = L;
      }
    }
  }
}

// Merge the split partials of one query head (fixed order):
//   M = max m_s,  L = sum l_s e^(m_s - M),  out = sum o_s e^(m_s - M) / L.
// One workgroup per head; the split axis is spread over the threads so the
// loads are independent.
template <int HD, bool OF32>
__global__ void __launch_bounds__(kAttnBlock) attn_merge_kernel(AttnParams p) {
  constexpr int SUB = kAttnBlock / HD * 4;  // split lanes per column (4 columns per thread)
  __shared__ float wsh[CPI_ATTN_MAX_SPLITS];
  __shared__ float red[kAttnWaves];
  __shared__ float part[SUB][HD];
  const int h = blockIdx.x;
  int seq = p.position ? (*p.position + 1) : p.seq_len;
  if (seq > p.max_ctx) seq = p.max_ctx;
  const int start = (p.window > 0 && seq > p.window) ? seq - p.window : 0;
  const int len = seq - start;
  constexpr int CT = (kAttnBlock / (HD / 8)) * 2;
  int chunk = (len + p.nsplit - 1) / p.nsplit;
  chunk = ((chunk + CT - 1) / CT) * CT;
  if (chunk < CT) chunk = CT;
  const int active = (len + chunk - 1) / chunk;
  if (active <= 1) return;  // the split kernel already wrote the output
  const size_t maxs = CPI_ATTN_MAX_SPLITS;
  const float* ml = p.scratch + kCounterSlots + static_cast<size_t>(h) * maxs * 2;
  const float* os = p.scratch + kCounterSlots + static_cast<size_t>(p.nh) * maxs * 2 +
                    static_cast<size_t>(h) * maxs * HD;
  const int tid = threadIdx.x;
  float mv = -INFINITY;
  if (tid < active) mv = ml[2 * tid];
  // block max of m
  float M = wave_max(mv);
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = M;
  __syncthreads();
  M = red[0];
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, red[w]);
  __syncthreads();
  float lw = 0.f;
  if (tid < active) {
    const float w = safe_exp_diff(mv, M);
    wsh[tid] = w;
    lw = ml[2 * tid + 1] * w;
  }
  const float L = block_sum(lw, red);  // includes a barrier: wsh is visible
  // columns: thread handles 4 consecutive columns for splits s = sub, sub+SUB, ...
  const int c4 = (tid % (HD / 4)) * 4;
  const int sub = tid / (HD / 4);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s2 = sub; s2 < active; s2 += SUB) {
    const float w = wsh[s2];
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 v = *reinterpret_cast<const f32x4*>(os + static_cast<size_t>(s2) * HD + c4);
    acc[0] = fmaf(v.x, w, acc[0]);
    acc[1] = fmaf(v.y, w, acc[1]);
    acc[2] = fmaf(v.z, w, acc[2]);
    acc[3] = fmaf(v.w, w, acc[3]);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) part[sub][c4 + e] = acc[e];
  __syncthreads();
  if (tid < HD) {
    float r = 0.f;
#pragma unroll
    for (int q = 0; q < SUB; ++q) r += part[q][tid];
    r /= L;
    if (OF32) static_cast<float*>(p.out)[h * HD + tid] = r;
    else static_cast<uint16_t*>(p.out)[h * HD + tid] = f2h(r);
  }
}

namespace {

template <int HD, int G>
hipError_t launch_g(const AttnParams& p, bool qf32, bool of32, hipStream_t s) {
  dim3 grid(p.nkv, p.nsplit);
  if (qf32 && of32) hipLaunchKernelGGL((attn_kernel<HD, G, true, true>), grid, dim3(kAttnBlock), 0, s, p);
  else if (qf32) hipLaunchKernelGGL((attn_kernel<HD, G, true, false>), grid, dim3(kAttnBlock), 0, s, p);
  else if (of32) hipLaunchKernelGGL((attn_kernel<HD, G, false, true>), grid, dim3(kAttnBlock), 0, s, p);
  else hipLaunchKernelGGL((attn_kernel<HD, G, false, false>), grid, dim3(kAttnBlock), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (of32) hipLaunchKernelGGL((attn_merge_kernel<HD, true>), dim3(p.nh), dim3(kAttnBlock), 0, s, p);
  else hipLaunchKernelGGL((attn_merge_kernel<HD, false>), dim3(p.nh), dim3(kAttnBlock), 0, s, p);
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
  int n = 512 / (nkv > 0 ? nkv : 1);
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

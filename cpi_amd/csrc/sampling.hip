// On-device sampling for the decode graph: the resident engine's sampler
// (src/engine/llama_engine_sampling_utils.cpp:10-189, sample_from_logits) run
// by one workgroup on the device logits, so a sampled token costs no logits
// copy to the host (the reference's logits graph copies all V floats per
// token, src/engine/llama_engine_graph.cpp:818-837).  The uniform draw r of
// each step comes from a small device array the host fills from the same
// generator the reference samples with (mt19937(42), one float per token).
//
// Thread t of 512 owns the contiguous logits [t*EPT, (t+1)*EPT) in registers
// (EPT 64 or 128: vocabularies up to 65536).
//   1. non-finite -> -inf, clamp to [-80, 80]; repetition penalty on ids set
//      in the `seen` bitmap (the distinct history ids); no-repeat n-gram bans
//      from the history array into an LDS bitmap.
//   2. temperature <= 0: first maximum.
//   3. s = l * (1/T); max over finite s.
//   4. top-k: the k-th largest s by a 4-pass MSB radix select on
//      order-preserving 32-bit keys; s below it -> -inf (ties kept).
//   5. p = exp(s - max) / sum.
//   6. top-p: the largest threshold T with sum(p >= T) >= top_p, found by
//      bisection on the bit patterns of positive floats (deterministic block
//      sums); p < T -> 0, renormalise.  Equals the reference's sorted prefix
//      up to the order of equal probabilities.
//   7. the first id whose inclusive cumulative probability reaches r (block
//      exclusive scan of per-thread sums), else the first most probable id.
// Then the greedy loop's bookkeeping: *token, ring[*step % ring_len],
// ++*step, ++*position, the seen bit and history[*position] of the new token.
// Floating-point sums are blocked (per thread, then across threads) where the
// reference sums in index order: picks can differ only when r falls within a
// few ulps of a cumulative boundary.
#include "common.hpp"
#include "../../include/cpi_hip.h"

namespace cpi {

constexpr int kSampThreads = 512;
constexpr int kSampWaves = kSampThreads / kWave;
constexpr int kSampMaxVocab = kSampThreads * 128;

struct SampleParams {
  float temperature;
  int top_k;
  float top_p;
  float rep_penalty;
  int ngram;
};

// Order-preserving key of a float: a < b  <=>  fkey(a) < fkey(b) (-inf lowest).
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float samp_sum(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kSampWaves; ++w) s += red[w];
  __syncthreads();
  return s;
}

__device__ __forceinline__ float samp_max(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kSampWaves; ++w) m = fmaxf(m, red[w]);
  __syncthreads();
  return m;
}

__device__ __forceinline__ int samp_min_int(int v, int* red) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v = min(v, __shfl_xor(v, m, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  int r = red[0];
#pragma unroll
  for (int w = 1; w < kSampWaves; ++w) r = min(r, red[w]);
  __syncthreads();
  return r;
}

// First maximum: (value, index) with ties to the lower index.
__device__ __forceinline__ int samp_argmax(float v, int i, float* redv, int* redi) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float ov = __shfl_xor(v, m, kWave);
    const int oi = __shfl_xor(i, m, kWave);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
  }
  if ((threadIdx.x & (kWave - 1)) == 0) {
    redv[threadIdx.x / kWave] = v;
    redi[threadIdx.x / kWave] = i;
  }
  __syncthreads();
  float bv = redv[0];
  int bi = redi[0];
#pragma unroll
  for (int w = 1; w < kSampWaves; ++w)
    if (redv[w] > bv || (redv[w] == bv && redi[w] < bi)) { bv = redv[w]; bi = redi[w]; }
  __syncthreads();
  return bi;
}

// Exclusive prefix sum of one float per thread, in thread order.
__device__ __forceinline__ float samp_exclusive_scan(float v, float* red) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  float inc = v;
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float o = __shfl_up(inc, m, kWave);
    if (lane >= m) inc += o;
  }
  if (lane == kWave - 1) red[wave] = inc;
  __syncthreads();
  float base = 0.f;
  for (int w = 0; w < wave; ++w) base += red[w];
  __syncthreads();
  return base + inc - v;
}

template <int EPT>
__global__ void __launch_bounds__(kSampThreads) sample_advance_kernel(
    const float* logits, int V, SampleParams sp, const float* rand, int rand_len, uint32_t* seen, int* history,
    int hist_cap, int* token, int* position, int* step, int* ring, int ring_len) {
  __shared__ uint32_t ban[kSampMaxVocab / 32];
  __shared__ float redf[kSampWaves];
  __shared__ int redi[kSampWaves];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sel_prefix, sel_k;

  const int t = threadIdx.x;
  const int i0 = t * EPT;
  const int pos = *position;
  const int st = *step;
  const int hist_len = history ? min(pos + 1, hist_cap) : 0;

  // ---- 1. n-gram bans (llama_engine_sampling_utils.cpp:55-94)
  const bool ngram = sp.ngram > 1 && history && hist_len + 1 >= sp.ngram;
  if (ngram) {
    for (int w = t; w < (V + 31) / 32; w += kSampThreads) ban[w] = 0u;
    __syncthreads();
    const int pre = sp.ngram - 1;
    for (int i = t; i + sp.ngram <= hist_len; i += kSampThreads) {
      bool match = true;
      for (int j = 0; j < pre && match; ++j) match = history[i + j] == history[hist_len - pre + j];
      if (match) {
        const int nx = history[i + pre];
        if (nx >= 0 && nx < V) atomicOr(&ban[nx >> 5], 1u << (nx & 31));
      }
    }
    __syncthreads();
  }

  float v[EPT];
  bool cand = false;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = i0 + e;
    float x = -INFINITY;
    if (i < V) {
      x = logits[i];
      x = isfinite(x) ? fminf(fmaxf(x, -80.f), 80.f) : -INFINITY;
      if (sp.rep_penalty > 1.f && seen && ((seen[i >> 5] >> (i & 31)) & 1u))
        x = x > 0.f ? x / sp.rep_penalty : x * sp.rep_penalty;
      if (ngram && ((ban[i >> 5] >> (i & 31)) & 1u)) x = -INFINITY;
      cand |= isfinite(x);
    }
    v[e] = x;
  }
  int pick = -1;
  if (ngram && samp_max(cand ? 1.f : 0.f, redf) == 0.f) pick = 0;  // every id banned (:88-93)

  if (pick < 0 && sp.temperature <= 0.f) {
    // ---- 2. first maximum
    float bv = -INFINITY;
    int bi = INT32_MAX;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (i0 + e < V && (v[e] > bv || bi == INT32_MAX)) { bv = v[e]; bi = i0 + e; }
    pick = samp_argmax(bv, bi, redf, redi);
  } else if (pick < 0) {
    // ---- 3. temperature and max over finite
    const float inv_t = 1.f / sp.temperature;
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      v[e] = v[e] * inv_t;
      if (isfinite(v[e])) mx = fmaxf(mx, v[e]);
    }
    mx = samp_max(mx, redf);
    if (!isfinite(mx)) {
      pick = 0;
    } else {
      // ---- 4. top-k: k-th largest key, MSB-first radix select
      if (sp.top_k > 0 && sp.top_k < V) {
        if (t == 0) {
          sel_prefix = 0u;
          sel_k = static_cast<uint32_t>(sp.top_k);
        }
        uint32_t mask = 0u;
        for (int shift = 24; shift >= 0; shift -= 8) {
          if (t < 256) hist[t] = 0u;
          __syncthreads();
          const uint32_t prefix = sel_prefix;
#pragma unroll
          for (int e = 0; e < EPT; ++e) {
            if (i0 + e >= V) continue;
            const uint32_t key = fkey(v[e]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
          }
          __syncthreads();
          if (t == 0) {
            uint32_t k = sel_k, d = 255u;
            for (;; --d) {
              if (hist[d] >= k || d == 0u) break;
              k -= hist[d];
            }
            sel_k = k;
            sel_prefix = prefix | (d << shift);
          }
          mask |= 255u << shift;
          __syncthreads();
        }
        const uint32_t kth = sel_prefix;
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (fkey(v[e]) < kth) v[e] = -INFINITY;
      }
      // ---- 5. softmax
      float local = 0.f;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        v[e] = isfinite(v[e]) ? expf(v[e] - mx) : 0.f;
        local += v[e];
      }
      const float sum = samp_sum(local, redf);
      if (!(sum > 0.f)) {
        pick = 0;
      } else {
        float pmax = 0.f;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          v[e] = v[e] / sum;
          pmax = fmaxf(pmax, v[e]);
        }
        // ---- 6. top-p threshold by bisection over positive float bits
        if (sp.top_p > 0.f && sp.top_p < 1.f) {
          pmax = samp_max(pmax, redf);
          uint32_t lo = 1u, hi = __float_as_uint(pmax);
          while (lo < hi) {
            const uint32_t mid = lo + (hi - lo + 1u) / 2u;
            const float thr = __uint_as_float(mid);
            float part = 0.f;
#pragma unroll
            for (int e = 0; e < EPT; ++e) part += v[e] >= thr ? v[e] : 0.f;
            if (samp_sum(part, redf) >= sp.top_p) lo = mid;
            else hi = mid - 1u;
          }
          const float thr = __uint_as_float(lo);
          float kept = 0.f;
#pragma unroll
          for (int e = 0; e < EPT; ++e) {
            v[e] = v[e] >= thr ? v[e] : 0.f;
            kept += v[e];
          }
          const float renorm = samp_sum(kept, redf);
          if (renorm > 0.f) {
#pragma unroll
            for (int e = 0; e < EPT; ++e) v[e] = v[e] / renorm;
          }
        }
        // ---- 7. inverse CDF at r
        const float r = rand[st % rand_len];
        float own = 0.f;
#pragma unroll
        for (int e = 0; e < EPT; ++e) own += v[e];
        float acc = samp_exclusive_scan(own, redf);
        int first = INT32_MAX;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          if (i0 + e >= V) break;
          acc += v[e];
          if (first == INT32_MAX && r <= acc) first = i0 + e;
        }
        pick = samp_min_int(first, redi);
        if (pick == INT32_MAX) {
          float bv = -1.f;
          int bi = INT32_MAX;
#pragma unroll
          for (int e = 0; e < EPT; ++e)
            if (i0 + e < V && v[e] > bv) { bv = v[e]; bi = i0 + e; }
          pick = samp_argmax(bv, bi, redf, redi);
        }
      }
    }
  }

  if (t == 0) {
    *token = pick;
    ring[st % ring_len] = pick;
    *step = st + 1;
    *position = pos + 1;
    if (seen && pick >= 0 && pick < V) seen[pick >> 5] |= 1u << (pick & 31);
    if (history && pos + 1 < hist_cap) history[pos + 1] = pick;
  }
}

hipError_t sample_advance_launch(const float* logits, int V, const SampleParams& sp, const float* rand, int rand_len,
                                 uint32_t* seen, int* history, int hist_cap, int* token, int* position, int* step,
                                 int* ring, int ring_len, hipStream_t s) {
  const dim3 g(1), b(kSampThreads);
  if (V <= kSampThreads * 64)
    hipLaunchKernelGGL(sample_advance_kernel<64>, g, b, 0, s, logits, V, sp, rand, rand_len, seen, history,
                       hist_cap, token, position, step, ring, ring_len);
  else if (V <= kSampMaxVocab)
    hipLaunchKernelGGL(sample_advance_kernel<128>, g, b, 0, s, logits, V, sp, rand, rand_len, seen, history,
                       hist_cap, token, position, step, ring, ring_len);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace cpi

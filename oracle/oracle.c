/*
 * oracle.c — CPU restatement of kurulav1/cpi's reference CPU decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the CPU baseline timed by bench.py; nothing in the product links or
 * calls it.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * What it follows (file:line in /root/reference):
 *   .ll2c header V1-V4 + tensor table ........ src/model/weight_loader.cpp:10-242
 *   fp16 -> fp32 .............................. src/engine/cpu_engine.cpp:71-94
 *   gemv (8-lane fp32 FMA + hsum256 order) .... src/engine/cpu_engine.cpp:134-184,325-385
 *   int8 / int4 dequant (row / global scale) .. src/engine/cpu_engine.cpp:855-914
 *   RMSNorm / LayerNorm ....................... src/engine/cpu_engine.cpp:392-424
 *   rotate-half RoPE from fp32 tables ......... src/engine/cpu_engine.cpp:429-447,1033-1045
 *   attention (fp32 KV, 2-pass softmax) ....... src/engine/cpu_engine.cpp:451-523
 *   SwiGLU MLP ................................ src/engine/cpu_engine.cpp:531-559
 *   MoE router + experts ...................... src/engine/cpu_engine.cpp:561-637
 *   forward_token ............................. src/engine/cpu_engine.cpp:650-706
 *   greedy (first max) ........................ src/engine/cpu_engine.cpp:726-729
 *   sampling (GPU engine's sampler) ........... src/engine/llama_engine_sampling_utils.cpp:10-189
 *   generate_stream ........................... src/engine/cpu_engine.cpp:1064-1126
 *
 * Deliberate, documented deviations from the reference CPU engine:
 *   - RoPE uses the file's effective theta (rope_theta or family default), the
 *     value the GPU engine uses (llama_engine_lifecycle.cpp:277-284); the CPU
 *     engine hardcodes 10000 (cpu_engine.cpp:1037).  Identical for theta 1e4.
 *   - Attention projections may also be stored low-bit (the CPU engine only
 *     accepts fp16 wq/wk/wv/wo, cpu_engine.cpp:933-936).
 *   - Extension format: "<name>.int4" + "<name>.gscale" = int4 with one fp16
 *     scale per 32 consecutive columns (BASELINE group-32 configs).
 *   - EOS may be disabled (eos < 0) so random-init greedy runs are not cut.
 *   - Low-bit rows are dequantised per row on the fly instead of once at init;
 *     the dequantised values and the summation order are the same.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define ORACLE_AVX2 1
#endif

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ fp16 */
EXPORT float oracle_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t e = (h >> 10) & 0x1F;
  const uint32_t m = h & 0x3FF;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      uint32_t mm = m, k = 0;
      while (!(mm & 0x400)) { mm <<= 1; ++k; }
      bits = sign | ((127 - 15 - k + 1) << 23) | ((mm & 0x3FF) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Nibble decode of the packed int4 format: low nibble = even column,
 * two's complement (kernels_weight_only_matvec.cu:35-43, cpu_engine.cpp:876-881). */
EXPORT int oracle_int4_nibble(uint8_t byte, int high) {
  const uint8_t nib = high ? (uint8_t)((byte >> 4) & 0x0F) : (uint8_t)(byte & 0x0F);
  return nib >= 8 ? (int)nib - 16 : (int)nib;
}

/* ------------------------------------------------------------ matrices */
enum { OW_F16 = 0, OW_I8ROW = 1, OW_I4ROW = 2, OW_I4G32 = 3, OW_F32 = 4 };

typedef struct {
  int fmt;
  const void* w;
  const void* scales;
  long scale_count;
  int R, K;
} omat;

/* Dequantised fp32 value row r (length K) into dst. */
static void mat_row(const omat* m, int r, float* dst) {
  const int K = m->K;
  switch (m->fmt) {
    case OW_F16: {
      const uint16_t* row = (const uint16_t*)m->w + (size_t)r * K;
      int j = 0;
#ifdef ORACLE_AVX2
      /* F16C conversion is exact, identical to oracle_fp16_to_fp32 */
      for (; j + 8 <= K; j += 8)
        _mm256_storeu_ps(dst + j, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(row + j))));
#endif
      for (; j < K; ++j) dst[j] = oracle_fp16_to_fp32(row[j]);
      break;
    }
    case OW_F32:
      memcpy(dst, (const float*)m->w + (size_t)r * K, sizeof(float) * K);
      break;
    case OW_I8ROW: {
      const float* sc = (const float*)m->scales;
      const float s = m->scale_count > 1 ? sc[r] : sc[0];
      const int8_t* row = (const int8_t*)m->w + (size_t)r * K;
      for (int j = 0; j < K; ++j) dst[j] = (float)row[j] * s;
      break;
    }
    case OW_I4ROW: {
      const float* sc = (const float*)m->scales;
      const float s = m->scale_count > 1 ? sc[r] : sc[0];
      const int pc = (K + 1) / 2;
      const uint8_t* row = (const uint8_t*)m->w + (size_t)r * pc;
      for (int j = 0; j < K; ++j) dst[j] = (float)oracle_int4_nibble(row[j / 2], j & 1) * s;
      break;
    }
    case OW_I4G32: {
      const int pc = (K + 1) / 2;
      const int ng = (K + 31) / 32;
      const uint8_t* row = (const uint8_t*)m->w + (size_t)r * pc;
      const uint16_t* gs = (const uint16_t*)m->scales + (size_t)r * ng;
      int j = 0;
#ifdef ORACLE_AVX2
      /* 8 columns at a time: sign-extend nibbles, times the group scale */
      for (; j + 8 <= K; j += 8) {
        const uint32_t b4 = (uint32_t)row[j / 2] | ((uint32_t)row[j / 2 + 1] << 8) |
                            ((uint32_t)row[j / 2 + 2] << 16) | ((uint32_t)row[j / 2 + 3] << 24);
        const __m256i sh = _mm256_setr_epi32(28, 24, 20, 16, 12, 8, 4, 0);
        const __m256i q = _mm256_srai_epi32(_mm256_sllv_epi32(_mm256_set1_epi32((int)b4), sh), 28);
        const __m256 s = _mm256_set1_ps(oracle_fp16_to_fp32(gs[j / 32]));
        _mm256_storeu_ps(dst + j, _mm256_mul_ps(_mm256_cvtepi32_ps(q), s));
      }
#endif
      for (; j < K; ++j)
        dst[j] = (float)oracle_int4_nibble(row[j / 2], j & 1) * oracle_fp16_to_fp32(gs[j / 32]);
      break;
    }
  }
}

/* Dot of an fp32 row with x using the reference's 8-lane FMA accumulation and
 * its hsum256 reduction order ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)). */
static float dot8(const float* w, const float* x, int K) {
  const int K8 = K & ~7;
#ifdef ORACLE_AVX2
  __m256 acc = _mm256_setzero_ps();
  for (int j = 0; j < K8; j += 8)
    acc = _mm256_fmadd_ps(_mm256_loadu_ps(w + j), _mm256_loadu_ps(x + j), acc);
  float a[8];
  _mm256_storeu_ps(a, acc);
#else
  float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < K8; j += 8)
    for (int l = 0; l < 8; ++l) a[l] = fmaf(w[j + l], x[j + l], a[l]);
#endif
  for (int j = K8; j < K; ++j) a[j - K8] = fmaf(w[j], x[j], a[j - K8]); /* zero-padded tail */
  const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
  return (s0 + s1) + (s2 + s3);
}

EXPORT void oracle_gemv(int fmt, const void* w, const void* scales, long scale_count, int R, int K,
                        const float* x, float* y) {
  omat m = {fmt, w, scales, scale_count, R, K};
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(dynamic, 16)
    for (int r = 0; r < R; ++r) {
      mat_row(&m, r, row);
      y[r] = dot8(row, x, K);
    }
    free(row);
  }
}

/* -------------------------------------------------------- small kernels */
EXPORT void oracle_rmsnorm(const float* x, const uint16_t* w, const uint16_t* b, float eps,
                           int layernorm, float* out, int n) {
  if (layernorm) {
    float sum = 0.f, sq = 0.f;
    for (int i = 0; i < n; ++i) { sum += x[i]; sq += x[i] * x[i]; }
    const float mean = sum / (float)n;
    float var = sq / (float)n - mean * mean;
    if (var < 0.f) var = 0.f;
    const float inv = 1.0f / sqrtf(var + eps);
    for (int i = 0; i < n; ++i)
      out[i] = (x[i] - mean) * inv * oracle_fp16_to_fp32(w[i]) + (b ? oracle_fp16_to_fp32(b[i]) : 0.f);
    return;
  }
  float ss = 0.f;
  for (int i = 0; i < n; ++i) ss += x[i] * x[i];
  const float rms = 1.f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i)
    out[i] = rms * x[i] * oracle_fp16_to_fp32(w[i]) + (b ? oracle_fp16_to_fp32(b[i]) : 0.f);
}

EXPORT void oracle_rope_tables(int max_ctx, int hd, float theta, float* cos_t, float* sin_t) {
  const int half = hd / 2;
  for (int p = 0; p < max_ctx; ++p)
    for (int d = 0; d < half; ++d) {
      const float freq = 1.f / powf(theta, (float)(2 * d) / (float)hd);
      cos_t[(size_t)p * half + d] = cosf((float)p * freq);
      sin_t[(size_t)p * half + d] = sinf((float)p * freq);
    }
}

EXPORT void oracle_rope(float* q, float* k, int pos, int nh, int nkv, int hd, const float* cos_t,
                        const float* sin_t) {
  const int half = hd / 2;
  const float* c = cos_t + (size_t)pos * half;
  const float* s = sin_t + (size_t)pos * half;
  for (int h = 0; h < nh + nkv; ++h) {
    float* v = h < nh ? q + (size_t)h * hd : k + (size_t)(h - nh) * hd;
    for (int d = 0; d < half; ++d) {
      const float x0 = v[d], x1 = v[d + half];
      v[d] = x0 * c[d] - x1 * s[d];
      v[d + half] = x0 * s[d] + x1 * c[d];
    }
  }
}

/* Attention of one token over caches [ctx, kvdim] (fp32) for positions
 * [start, seq); scores scratch nh*ctx. */
EXPORT void oracle_attention(const float* q, const float* kc, const float* vc, int seq, int window,
                             int nh, int nkv, int hd, float* out, float* scores) {
  const int kv_mul = nh / nkv;
  const int kvdim = nkv * hd;
  const float scale = 1.f / sqrtf((float)hd);
  const int len = (window > 0 && window < seq) ? window : seq;
  const int start = seq - len;
#pragma omp parallel for schedule(dynamic, 1)
  for (int h = 0; h < nh; ++h) {
    const int hk = h / kv_mul;
    const float* qh = q + (size_t)h * hd;
    float* sc = scores + (size_t)h * seq;
    for (int t = 0; t < len; ++t) {
      const float* kt = kc + (size_t)(start + t) * kvdim + (size_t)hk * hd;
      float dot = 0.f;
      for (int d = 0; d < hd; ++d) dot += qh[d] * kt[d];
      sc[t] = dot * scale;
    }
    float mx = sc[0];
    for (int t = 1; t < len; ++t) if (sc[t] > mx) mx = sc[t];
    float sum = 0.f;
    for (int t = 0; t < len; ++t) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
    const float inv = 1.f / sum;
    for (int t = 0; t < len; ++t) sc[t] *= inv;
    float* oh = out + (size_t)h * hd;
    for (int d = 0; d < hd; ++d) oh[d] = 0.f;
    for (int t = 0; t < len; ++t) {
      const float* vt = vc + (size_t)(start + t) * kvdim + (size_t)hk * hd;
      const float a = sc[t];
      for (int d = 0; d < hd; ++d) oh[d] += a * vt[d];
    }
  }
}

EXPORT float oracle_silu(float g) { return g / (1.f + expf(-g)); }

EXPORT void oracle_router_topk(const float* logits, int experts, int top_k, int* idx, float* prob) {
  float* p = (float*)malloc(sizeof(float) * (size_t)experts);
  char* used = (char*)calloc((size_t)experts, 1);
  float mx = logits[0];
  for (int i = 1; i < experts; ++i) mx = fmaxf(mx, logits[i]);
  float sum = 0.f;
  for (int i = 0; i < experts; ++i) { p[i] = expf(logits[i] - mx); sum += p[i]; }
  const float inv = 1.f / fmaxf(sum, 1e-8f);
  for (int i = 0; i < experts; ++i) p[i] *= inv;
  float ps = 0.f;
  for (int k = 0; k < top_k; ++k) {
    int best = -1;
    float bp = -1.f;
    for (int e = 0; e < experts; ++e) {
      if (used[e]) continue;
      if (p[e] > bp) { best = e; bp = p[e]; }
    }
    idx[k] = best < 0 ? 0 : best;
    prob[k] = bp > 0.f ? bp : 0.f;
    if (best >= 0) used[best] = 1;
    ps += prob[k];
  }
  const float ip = 1.f / fmaxf(ps, 1e-8f);
  for (int k = 0; k < top_k; ++k) prob[k] *= ip;
  free(p);
  free(used);
}

EXPORT int oracle_argmax(const float* x, int n) {
  int best = 0;
  for (int i = 1; i < n; ++i) if (x[i] > x[best]) best = i;
  return best;
}

/* ----------------------------------------------------------- sampling
 * The resident engine's sampler, src/engine/llama_engine_sampling_utils.cpp:
 * 10-189 (sample_from_logits), in float as there, with the uniform draw r in
 * [0, 1) passed in (the reference draws it from a thread-local mt19937(42)).
 * Steps: non-finite -> -inf and clamp to [-80, 80] (:26-35); repetition
 * penalty over the distinct history ids (:37-49); no-repeat n-gram bans
 * (:55-94); temperature <= 0 -> first max (:96-98); scale by 1/T and max over
 * finite (:100-113); top-k keeps values >= the k-th largest (:115-124);
 * softmax (:126-139); top-p keeps the most probable ids until their sum
 * reaches top_p, then renormalises (:141-171); first i with r <= cumulative
 * probability, else the most probable id (:173-188).  Ties in the top-p
 * order (unspecified under std::sort) are broken by lower id first.
 * `logits` is modified.  Returns the sampled id. */
static const float* g_sort_probs;
static int cmp_prob_desc(const void* a, const void* b) {
  const int i = *(const int*)a, j = *(const int*)b;
  const float pi = g_sort_probs[i], pj = g_sort_probs[j];
  if (pi > pj) return -1;
  if (pi < pj) return 1;
  return i < j ? -1 : (i > j);
}
static int cmp_float_desc(const void* a, const void* b) {
  const float x = *(const float*)a, y = *(const float*)b;
  return x > y ? -1 : (x < y);
}

EXPORT int oracle_sample(float* logits, int V, float temperature, int top_k, float top_p, float rep_penalty,
                         int ngram, const int* history, int hist_len, float r) {
  if (V <= 0) return 0;
  for (int i = 0; i < V; ++i) {
    float v = logits[i];
    if (!isfinite(v)) { logits[i] = -INFINITY; continue; }
    logits[i] = v > 80.f ? 80.f : (v < -80.f ? -80.f : v);
  }
  if (rep_penalty > 1.f && hist_len > 0) {
    char* seen = (char*)calloc((size_t)V, 1);
    for (int h = 0; h < hist_len; ++h) {
      const int id = history[h];
      if (id < 0 || id >= V || seen[id]) continue;
      seen[id] = 1;
      logits[id] = logits[id] > 0.f ? logits[id] / rep_penalty : logits[id] * rep_penalty;
    }
    free(seen);
  }
  if (ngram > 1 && hist_len + 1 >= ngram) {
    const int pre = ngram - 1;
    char* banned = (char*)calloc((size_t)V, 1);
    for (int i = 0; i + ngram <= hist_len; ++i) {
      int match = 1;
      for (int j = 0; j < pre; ++j)
        if (history[i + j] != history[hist_len - pre + j]) { match = 0; break; }
      if (match) {
        const int nx = history[i + pre];
        if (nx >= 0 && nx < V) banned[nx] = 1;
      }
    }
    int cand = 0;
    for (int i = 0; i < V; ++i) {
      if (banned[i]) logits[i] = -INFINITY;
      else if (isfinite(logits[i])) cand = 1;
    }
    free(banned);
    if (!cand) return 0;
  }
  if (temperature <= 0.f) {
    int best = 0;
    for (int i = 1; i < V; ++i) if (logits[i] > logits[best]) best = i;
    return best;
  }
  const float inv_t = 1.f / temperature;
  float mx = -INFINITY;
  for (int i = 0; i < V; ++i)
    if (isfinite(logits[i])) { const float s = logits[i] * inv_t; if (s > mx) mx = s; }
  if (!isfinite(mx)) return 0;
  for (int i = 0; i < V; ++i) logits[i] = logits[i] * inv_t;
  if (top_k > 0 && top_k < V) {
    float* copy = (float*)malloc(sizeof(float) * (size_t)V);
    memcpy(copy, logits, sizeof(float) * (size_t)V);
    qsort(copy, (size_t)V, sizeof(float), cmp_float_desc);
    const float kth = copy[top_k - 1];
    free(copy);
    for (int i = 0; i < V; ++i) if (logits[i] < kth) logits[i] = -INFINITY;
  }
  float* p = (float*)calloc((size_t)V, sizeof(float));
  float sum = 0.f;
  for (int i = 0; i < V; ++i) {
    if (!isfinite(logits[i])) continue;
    p[i] = expf(logits[i] - mx);
    sum += p[i];
  }
  if (sum <= 0.f) { free(p); return 0; }
  for (int i = 0; i < V; ++i) p[i] /= sum;
  if (top_p > 0.f && top_p < 1.f) {
    int* idx = (int*)malloc(sizeof(int) * (size_t)V);
    char* keep = (char*)calloc((size_t)V, 1);
    for (int i = 0; i < V; ++i) idx[i] = i;
    g_sort_probs = p;
    qsort(idx, (size_t)V, sizeof(int), cmp_prob_desc);
    float cs = 0.f;
    for (int k = 0; k < V; ++k) {
      const int id = idx[k];
      if (p[id] <= 0.f) continue;
      keep[id] = 1;
      cs += p[id];
      if (cs >= top_p) break;
    }
    float rn = 0.f;
    for (int i = 0; i < V; ++i) { if (!keep[i]) p[i] = 0.f; rn += p[i]; }
    if (rn > 0.f) for (int i = 0; i < V; ++i) p[i] /= rn;
    free(idx);
    free(keep);
  }
  float acc = 0.f;
  int out = -1;
  for (int i = 0; i < V; ++i) {
    acc += p[i];
    if (r <= acc) { out = i; break; }
  }
  if (out < 0) {
    out = 0;
    for (int i = 1; i < V; ++i) if (p[i] > p[out]) out = i;
  }
  free(p);
  return out;
}

/* ------------------------------------------------------------- .ll2c file */
#pragma pack(push, 1)
typedef struct {
  char magic[8];
  int32_t version, vocab, hidden, inter, layers, heads;
} hdr_common;
typedef struct {
  char name[64];
  int64_t offset, bytes;
} tentry;
#pragma pack(pop)

typedef struct {
  int vocab, hidden, inter, layers, heads, kv_heads, max_seq;
  float rope_theta, norm_eps;
  int sliding_window, tie, qkv_bias, layernorm, family;
  int experts, experts_per_tok, expert_inter;
} ocfg;

typedef struct {
  uint8_t* base;
  size_t size;
  int count;
  const tentry* table;
  ocfg cfg;
} ofile;

static int file_open(ofile* f, const char* path) {
  memset(f, 0, sizeof(*f));
  int fd = open(path, O_RDONLY);
  if (fd < 0) return -1;
  struct stat st;
  if (fstat(fd, &st) != 0) { close(fd); return -1; }
  f->size = (size_t)st.st_size;
  f->base = (uint8_t*)mmap(NULL, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (f->base == MAP_FAILED) return -1;
  if (f->size < 48 || memcmp(f->base, "LL2CUDA", 7) != 0) return -2;
  int32_t v[20];
  memcpy(v, f->base + 8, sizeof(int32_t) * ((f->size - 8) / 4 < 20 ? (f->size - 8) / 4 : 20));
  const int version = v[0];
  ocfg* c = &f->cfg;
  c->vocab = v[1]; c->hidden = v[2]; c->inter = v[3]; c->layers = v[4]; c->heads = v[5];
  c->norm_eps = 1e-5f;
  int64_t table_off;
  if (version >= 2) {
    c->kv_heads = v[6]; c->max_seq = v[7];
    f->count = v[9];
    memcpy(&table_off, f->base + 8 + 4 * 10, 8);
    if (version >= 3) {
      const uint8_t* ext = f->base + 8 + 4 * 10 + 8;
      float rt, ne;
      int32_t sw, flags, fam;
      memcpy(&rt, ext, 4); memcpy(&ne, ext + 4, 4); memcpy(&sw, ext + 8, 4);
      memcpy(&flags, ext + 12, 4); memcpy(&fam, ext + 16, 4);
      c->rope_theta = rt;
      c->norm_eps = ne > 0.f ? ne : 1e-5f;
      c->sliding_window = sw;
      c->tie = flags & 1; c->qkv_bias = (flags >> 1) & 1; c->layernorm = (flags >> 2) & 1;
      c->family = fam;
      if (version >= 4) {
        int32_t e[3];
        memcpy(e, ext + 20, 12);
        c->experts = e[0]; c->experts_per_tok = e[1]; c->expert_inter = e[2];
      }
    }
  } else {
    c->kv_heads = v[5]; c->max_seq = v[6];
    f->count = v[8];
    memcpy(&table_off, f->base + 8 + 4 * 9, 8);
  }
  if (c->kv_heads <= 0 || c->heads <= 0 || c->heads % c->kv_heads) return -3;
  f->table = (const tentry*)(f->base + table_off);
  return 0;
}

static const tentry* file_find(const ofile* f, const char* name) {
  for (int i = 0; i < f->count; ++i)
    if (strncmp(f->table[i].name, name, 64) == 0) return &f->table[i];
  return NULL;
}

static float effective_theta(const ocfg* c) {
  if (c->rope_theta > 0.f) return c->rope_theta;
  if (c->family == 2) return 500000.f;
  if (c->family == 5) return 1000000.f;
  return 10000.f;
}

/* Binds "<name>" (fp16) or its low-bit variants. Returns 0 on success. */
static int bind_mat(const ofile* f, const char* name, int R, int K, omat* m) {
  char buf[96];
  const tentry* e = file_find(f, name);
  m->R = R; m->K = K; m->scales = NULL; m->scale_count = 0;
  if (e) { m->fmt = OW_F16; m->w = f->base + e->offset; return 0; }
  snprintf(buf, sizeof buf, "%s.int8", name);
  const tentry* q8 = file_find(f, buf);
  snprintf(buf, sizeof buf, "%s.int4", name);
  const tentry* q4 = file_find(f, buf);
  snprintf(buf, sizeof buf, "%s.gscale", name);
  const tentry* gs = file_find(f, buf);
  snprintf(buf, sizeof buf, "%s.scale", name);
  const tentry* sc = file_find(f, buf);
  if (q4 && gs) {
    m->fmt = OW_I4G32; m->w = f->base + q4->offset; m->scales = f->base + gs->offset;
    m->scale_count = gs->bytes / 2;
    return 0;
  }
  if (!sc || (!q8 && !q4)) return -1;
  m->scales = f->base + sc->offset;
  m->scale_count = sc->bytes / 4;
  if (q8) { m->fmt = OW_I8ROW; m->w = f->base + q8->offset; }
  else { m->fmt = OW_I4ROW; m->w = f->base + q4->offset; }
  return 0;
}

/* ---------------------------------------------------------------- engine */
typedef struct {
  const uint16_t *norm_att, *norm_ffn, *norm_att_b, *norm_ffn_b, *bo;
  omat wq, wk, wv, wo, w1, w2, w3, router;
  omat *ew1, *ew2, *ew3;
} olayer;

typedef struct {
  ofile f;
  ocfg c;
  int max_ctx, q_dim, hd, kv_dim;
  float theta;
  olayer* L;
  const uint16_t *emb, *norm_out, *norm_out_b, *lm_b;
  omat lm;
  float *x, *xn, *q, *k, *v, *att, *f1, *f2, *f3, *logits, *scores, *kc, *vc, *cos_t, *sin_t;
  float *moe_acc, *router_logits;
  char err[256];
} oengine;

static const uint16_t* opt16(const ofile* f, const char* name) {
  const tentry* e = file_find(f, name);
  return e ? (const uint16_t*)(f->base + e->offset) : NULL;
}

EXPORT void oracle_engine_free(oengine* e);

EXPORT oengine* oracle_engine_open(const char* path, int max_ctx, float theta_override) {
  oengine* e = (oengine*)calloc(1, sizeof(oengine));
  if (file_open(&e->f, path) != 0) { free(e); return NULL; }
  e->c = e->f.cfg;
  const ocfg* c = &e->c;
  e->max_ctx = max_ctx;
  e->theta = theta_override > 0.f ? theta_override : effective_theta(c);
  const int H = c->hidden, NL = c->layers;
  /* q_dim/head_dim from wq (fp16 bytes or low-bit rows) like cpu_engine.cpp:823-840 */
  omat probe;
  const tentry* wq = file_find(&e->f, "layers.0.attention.wq");
  if (wq) e->q_dim = (int)(wq->bytes / (2 * H));
  else {
    const tentry* s = file_find(&e->f, "layers.0.attention.wq.scale");
    const tentry* g = file_find(&e->f, "layers.0.attention.wq.gscale");
    e->q_dim = g ? (int)(g->bytes / 2 / ((H + 31) / 32)) : (s ? (int)(s->bytes / 4) : 0);
  }
  (void)probe;
  if (e->q_dim <= 0 || e->q_dim % c->heads) { oracle_engine_free(e); return NULL; }
  e->hd = e->q_dim / c->heads;
  e->kv_dim = c->kv_heads * e->hd;
  const int I = c->inter;
  const int EI = c->expert_inter > 0 ? c->expert_inter : I;
  const int FI = EI > I ? EI : I;
  e->emb = opt16(&e->f, "tok_embeddings.weight");
  e->norm_out = opt16(&e->f, "norm.weight");
  e->norm_out_b = opt16(&e->f, "norm.bias");
  e->lm_b = opt16(&e->f, "output.bias");
  if (!e->emb || !e->norm_out) { oracle_engine_free(e); return NULL; }
  if (bind_mat(&e->f, "output.weight", c->vocab, H, &e->lm) != 0) {
    e->lm.fmt = OW_F16; e->lm.w = e->emb; e->lm.R = c->vocab; e->lm.K = H;
  }
  e->L = (olayer*)calloc((size_t)NL, sizeof(olayer));
  char n[96];
  for (int l = 0; l < NL; ++l) {
    olayer* y = &e->L[l];
#define NM(s) (snprintf(n, sizeof n, "layers.%d.%s", l, s), n)
    y->norm_att = opt16(&e->f, NM("attention_norm.weight"));
    y->norm_ffn = opt16(&e->f, NM("ffn_norm.weight"));
    y->norm_att_b = opt16(&e->f, NM("attention_norm.bias"));
    y->norm_ffn_b = opt16(&e->f, NM("ffn_norm.bias"));
    y->bo = opt16(&e->f, NM("attention.bo"));
    int bad = !y->norm_att || !y->norm_ffn;
    bad |= bind_mat(&e->f, NM("attention.wq"), e->q_dim, H, &y->wq);
    bad |= bind_mat(&e->f, NM("attention.wk"), e->kv_dim, H, &y->wk);
    bad |= bind_mat(&e->f, NM("attention.wv"), e->kv_dim, H, &y->wv);
    bad |= bind_mat(&e->f, NM("attention.wo"), H, e->q_dim, &y->wo);
    if (c->experts <= 0) {
      bad |= bind_mat(&e->f, NM("feed_forward.w1"), I, H, &y->w1);
      bad |= bind_mat(&e->f, NM("feed_forward.w2"), H, I, &y->w2);
      bad |= bind_mat(&e->f, NM("feed_forward.w3"), I, H, &y->w3);
    } else {
      bad |= bind_mat(&e->f, NM("feed_forward.router"), c->experts, H, &y->router);
      y->ew1 = (omat*)calloc((size_t)c->experts, sizeof(omat));
      y->ew2 = (omat*)calloc((size_t)c->experts, sizeof(omat));
      y->ew3 = (omat*)calloc((size_t)c->experts, sizeof(omat));
      for (int x = 0; x < c->experts; ++x) {
        char b2[64];
        snprintf(b2, sizeof b2, "feed_forward.experts.%d.w1", x);
        bad |= bind_mat(&e->f, NM(b2), EI, H, &y->ew1[x]);
        snprintf(b2, sizeof b2, "feed_forward.experts.%d.w2", x);
        bad |= bind_mat(&e->f, NM(b2), H, EI, &y->ew2[x]);
        snprintf(b2, sizeof b2, "feed_forward.experts.%d.w3", x);
        bad |= bind_mat(&e->f, NM(b2), EI, H, &y->ew3[x]);
      }
    }
#undef NM
    if (bad) { oracle_engine_free(e); return NULL; }
  }
  const size_t kvn = (size_t)NL * max_ctx * e->kv_dim;
  e->x = calloc(H, 4); e->xn = calloc(H, 4); e->q = calloc(e->q_dim, 4);
  e->k = calloc(e->kv_dim, 4); e->v = calloc(e->kv_dim, 4); e->att = calloc(e->q_dim, 4);
  e->f1 = calloc(FI, 4); e->f2 = calloc(H, 4); e->f3 = calloc(FI, 4);
  e->logits = calloc(c->vocab, 4); e->scores = calloc((size_t)c->heads * max_ctx, 4);
  e->kc = calloc(kvn, 4); e->vc = calloc(kvn, 4);
  e->cos_t = calloc((size_t)max_ctx * (e->hd / 2), 4); e->sin_t = calloc((size_t)max_ctx * (e->hd / 2), 4);
  e->moe_acc = calloc(H, 4); e->router_logits = calloc(c->experts > 0 ? c->experts : 1, 4);
  if (!e->kc || !e->vc) { oracle_engine_free(e); return NULL; }
  oracle_rope_tables(max_ctx, e->hd, e->theta, e->cos_t, e->sin_t);
  return e;
}

EXPORT void oracle_engine_free(oengine* e) {
  if (!e) return;
  if (e->L) {
    for (int l = 0; l < e->c.layers; ++l) { free(e->L[l].ew1); free(e->L[l].ew2); free(e->L[l].ew3); }
    free(e->L);
  }
  free(e->x); free(e->xn); free(e->q); free(e->k); free(e->v); free(e->att); free(e->f1);
  free(e->f2); free(e->f3); free(e->logits); free(e->scores); free(e->kc); free(e->vc);
  free(e->cos_t); free(e->sin_t); free(e->moe_acc); free(e->router_logits);
  if (e->f.base) munmap(e->f.base, e->f.size);
  free(e);
}

EXPORT void oracle_engine_dims(const oengine* e, int* out) {
  out[0] = e->c.vocab; out[1] = e->c.hidden; out[2] = e->c.inter; out[3] = e->c.layers;
  out[4] = e->c.heads; out[5] = e->c.kv_heads; out[6] = e->hd; out[7] = e->max_ctx;
  out[8] = e->c.experts; out[9] = e->c.experts_per_tok;
}

static void gm(const omat* m, const float* x, float* y) {
  oracle_gemv(m->fmt, m->w, m->scales, m->scale_count, m->R, m->K, x, y);
}

static void mlp_dense(oengine* e, const olayer* y) {
  const int H = e->c.hidden, I = e->c.inter;
  gm(&y->w1, e->xn, e->f1);
  gm(&y->w3, e->xn, e->f3);
  for (int i = 0; i < I; ++i) e->f1[i] = oracle_silu(e->f1[i]) * e->f3[i];
  gm(&y->w2, e->f1, e->f2);
  for (int i = 0; i < H; ++i) e->x[i] += e->f2[i];
}

static void mlp_moe(oengine* e, const olayer* y) {
  const ocfg* c = &e->c;
  const int H = c->hidden;
  const int EI = c->expert_inter > 0 ? c->expert_inter : c->inter;
  int top_k = c->experts_per_tok > 0 ? c->experts_per_tok : 2;
  if (top_k > c->experts) top_k = c->experts;
  if (top_k < 1) top_k = 1;
  gm(&y->router, e->xn, e->router_logits);
  int idx[64];
  float pr[64];
  oracle_router_topk(e->router_logits, c->experts, top_k, idx, pr);
  memset(e->moe_acc, 0, sizeof(float) * H);
  for (int k = 0; k < top_k; ++k) {
    if (pr[k] <= 0.f) continue;
    const int x = idx[k];
    gm(&y->ew1[x], e->xn, e->f1);
    gm(&y->ew3[x], e->xn, e->f3);
    for (int i = 0; i < EI; ++i) e->f1[i] = oracle_silu(e->f1[i]) * e->f3[i];
    gm(&y->ew2[x], e->f1, e->f2);
    for (int i = 0; i < H; ++i) e->moe_acc[i] += pr[k] * e->f2[i];
  }
  for (int i = 0; i < H; ++i) e->x[i] += e->moe_acc[i];
}

/* One token at position pos; logits (fp32 [vocab]) copied to out if non-NULL. */
EXPORT int oracle_engine_forward(oengine* e, int token, int pos, float* out) {
  const ocfg* c = &e->c;
  const int H = c->hidden;
  if (pos < 0 || pos >= e->max_ctx || token < 0 || token >= c->vocab) return -1;
  const uint16_t* er = e->emb + (size_t)token * H;
  for (int i = 0; i < H; ++i) e->x[i] = oracle_fp16_to_fp32(er[i]);
  for (int l = 0; l < c->layers; ++l) {
    const olayer* y = &e->L[l];
    oracle_rmsnorm(e->x, y->norm_att, y->norm_att_b, c->norm_eps, c->layernorm, e->xn, H);
    gm(&y->wq, e->xn, e->q);
    gm(&y->wk, e->xn, e->k);
    gm(&y->wv, e->xn, e->v);
    oracle_rope(e->q, e->k, pos, c->heads, c->kv_heads, e->hd, e->cos_t, e->sin_t);
    const size_t lay = (size_t)l * e->max_ctx * e->kv_dim;
    memcpy(e->kc + lay + (size_t)pos * e->kv_dim, e->k, sizeof(float) * e->kv_dim);
    memcpy(e->vc + lay + (size_t)pos * e->kv_dim, e->v, sizeof(float) * e->kv_dim);
    oracle_attention(e->q, e->kc + lay, e->vc + lay, pos + 1, c->sliding_window, c->heads,
                     c->kv_heads, e->hd, e->att, e->scores);
    gm(&y->wo, e->att, e->f2);
    if (y->bo) for (int i = 0; i < H; ++i) e->f2[i] += oracle_fp16_to_fp32(y->bo[i]);
    for (int i = 0; i < H; ++i) e->x[i] += e->f2[i];
    oracle_rmsnorm(e->x, y->norm_ffn, y->norm_ffn_b, c->norm_eps, c->layernorm, e->xn, H);
    if (c->experts > 0) mlp_moe(e, y); else mlp_dense(e, y);
  }
  oracle_rmsnorm(e->x, e->norm_out, e->norm_out_b, c->norm_eps, c->layernorm, e->xn, H);
  gm(&e->lm, e->xn, e->logits);
  if (e->lm_b) for (int i = 0; i < c->vocab; ++i) e->logits[i] += oracle_fp16_to_fp32(e->lm_b[i]);
  if (out) memcpy(out, e->logits, sizeof(float) * c->vocab);
  return 0;
}

/* Greedy generate_stream (cpu_engine.cpp:1064-1126): forward every prompt
 * token, then sample(argmax) -> emit -> forward.  Writes up to max_new ids to
 * out_ids and, for the first n_logit_steps steps, the logits each id was
 * taken from (row-major [n_logit_steps, vocab]).  eos < 0 disables EOS.
 * Returns the number of ids generated. */
EXPORT int oracle_engine_generate(oengine* e, const int* prompt, int n_prompt, int max_new,
                                  int eos, int* out_ids, float* out_logits, int n_logit_steps) {
  int pos = 0;
  if (n_prompt <= 0) { oracle_engine_forward(e, 1, 0, NULL); pos = 1; }
  for (int i = 0; i < n_prompt && i < e->max_ctx; ++i) {
    if (oracle_engine_forward(e, prompt[i], i, NULL) != 0) return -1;
    pos = i + 1;
  }
  int n = 0;
  for (int step = 0; step < max_new; ++step) {
    if (out_logits && step < n_logit_steps)
      memcpy(out_logits + (size_t)step * e->c.vocab, e->logits, sizeof(float) * e->c.vocab);
    const int next = oracle_argmax(e->logits, e->c.vocab);
    out_ids[n++] = next;
    if (eos >= 0 && next == eos) break;
    if (pos >= e->max_ctx) break;
    oracle_engine_forward(e, next, pos++, NULL);
  }
  return n;
}

EXPORT int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

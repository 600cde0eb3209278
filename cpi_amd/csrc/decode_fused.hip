// Persistent fused decode step for gfx950: one launch runs a whole token —
// embedding, every layer (QKV GEMV + RMSNorm + RoPE + KV store, attention,
// o_proj + residual, w1|w3 + RMSNorm + SwiGLU, w2 + residual), the final
// norm + lm_head and the greedy argmax / token advance.
//
// Replaces the per-token launch sequence that the reference captures into
// its CUDA graph (src/engine/llama_engine_graph.cpp:166-480) — the same
// computation as cpi_hip_gemv / cpi_hip_attention_decode / cpi_hip_greedy_advance
// issued one kernel per op — for the resident int4-g32 path.
//
// Why one launch: at batch 1 every op is an HBM stream of a few to 50 MB, and
// a launch per op pays dispatch, ramp-up and tail each time (~3-5 us of a
// 5-12 us kernel).  Here the workgroups stay resident and meet at device-wide
// barriers between dependent phases; before waiting, each workgroup issues the
// weight loads of its first tile of the next phase (weights never depend on
// activations), so HBM keeps streaming across phase boundaries.
//
// Coherence: the XCDs' L2 caches are not coherent with each other, so every
// value produced and consumed inside the launch (residual x, q, attention
// output, SwiGLU output, logits, the current KV-cache row, attention partials)
// is written with device-coherent stores and read with device-coherent loads.
// Weights and older KV rows are read normally.
//
// Safety: every barrier wait is bounded.  A wait that exceeds the spin limit
// sets the abort word; every later barrier of the launch returns at once, so
// all waves reach the end of the kernel and the host reports the failure.
#include "common.hpp"
#include "gemv_plan.hpp"
#include "../../include/cpi_hip.h"

namespace cpi {

struct FusedParams {
  const cpi_fused_layer* layers;
  int nlayers;
  int H, I, V, nh, nkv, hd, max_ctx, window, nsplit;
  float eps, attn_scale;
  const uint16_t* emb;
  const uint16_t* norm_out;
  const uint16_t* lm_w;
  const float* rope_cos;
  const float* rope_sin;
  float* x;
  float* q;
  float* att;
  float* ff;
  float* logits;
  float* attn_scratch;
  int* token;
  int* pos;
  int* step;
  int* ring;
  int ring_len;
  uint32_t* sync;
  int spin_limit;
};

// sync words
constexpr int kSyncCount = 0;   // barrier arrivals (wraps; compared modulo 2^32)
constexpr int kSyncAbort = 1;   // non-zero: a barrier timed out
constexpr int kSyncBase = 2;    // arrival count at the start of the next launch
constexpr int kSyncArgmax = 4;  // u64 argmax key (words 4, 5)

// Tile configurations (rows per wave NR, passes per wave PP, K-split KS); a
// workgroup tile is NR * 4 / KS rows and covers the full row length.
template <int NR, int PP, int KS>
struct TileCfg {
  static constexpr int nr = NR, pp = PP, ks = KS;
  static constexpr int rb = NR * kWavesPerBlock / KS;  // rows per workgroup tile
  static_assert(NR * PP <= kMaxLoads, "loads per lane");
};
using CfgQKV = TileCfg<8, 2, 1>;  // 32 rows x K <= 4096 (int4 g32)
using CfgO = TileCfg<4, 1, 2>;    // 8 rows x K <= 4096
using CfgW13 = TileCfg<8, 2, 1>;  // 32 rows
using CfgW2 = TileCfg<4, 3, 2>;   // 8 rows x K <= 12288
using CfgLM = TileCfg<4, 4, 2>;   // 8 rows x K <= 4096 (fp16)

// Weight loads of one tile held in registers (16-byte chunks + group scales).
struct WBuf {
  u32x4 w[kMaxLoads];
  uint32_t s[kMaxLoads];  // GroupScales words of pass q at [q * nr, (q + 1) * nr)
};

// ---------------------------------------------------------------------------
// Device-wide barrier in two halves (bounded wait).  arrive: every thread's
// coherent stores have completed (vmcnt 0), then thread 0 counts the
// workgroup in.  The caller may then issue the next phase's weight loads;
// wait: thread 0 polls the count, and an LDS-only barrier releases the other
// waves without draining those loads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void barrier_arrive(const FusedParams& P, uint32_t& target, bool& live) {
  target += gridDim.x;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    live = coh_ld_u32(&P.sync[kSyncAbort]) == 0;
    if (live) __hip_atomic_fetch_add(&P.sync[kSyncCount], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ __forceinline__ void barrier_wait(const FusedParams& P, uint32_t target, bool live) {
  if (threadIdx.x == 0 && live) {
    int n = 0;
    while (static_cast<int32_t>(coh_ld_u32(&P.sync[kSyncCount]) - target) < 0) {
      if (++n > P.spin_limit) {
        coh_st_u32(&P.sync[kSyncAbort], 1u);
        break;
      }
      if ((n & 63) == 0 && coh_ld_u32(&P.sync[kSyncAbort]) != 0) break;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// GEMV tiles.
// ---------------------------------------------------------------------------
template <int FMT, class C>
__device__ __forceinline__ void tile_issue(const uint8_t* W, const uint16_t* S, int R, int K, int tile, WBuf& b) {
  const GemvPlan g = make_plan_nrpp(R, K, FmtT<FMT>::kElems, C::nr, C::pp, C::ks);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int rs = wave / C::ks, sg = wave % C::ks;
#pragma unroll
  for (int q = 0; q < C::pp; ++q) {
    const int pass = clamp_pass(g, sg, plan_pass(g, sg, 0, q));
    const int c = clamp_chunk(g, pass, lane);
    if constexpr (kGroupScaled<FMT>) {
      GroupScales<FMT, C::nr> gs;
      gs.load(S, g, plan_row(g, tile, rs, 0), c);
#pragma unroll
      for (int j = 0; j < static_cast<int>(sizeof(gs.w) / 4); ++j) b.s[q * C::nr + j] = gs.w[j];
    }
#pragma unroll
    for (int i = 0; i < C::nr; ++i) {
      const int row = clamp_row(g, plan_row(g, tile, rs, i));
      b.w[i * C::pp + q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(W + weight_offset(g, row, c)));
    }
  }
}

// Row sums of one tile into fin[0, RB) (LDS); every thread may read fin after.
template <int FMT, class C>
__device__ __forceinline__ void tile_compute(int R, int K, int tile, const WBuf& b, const uint32_t* prep,
                                             float* part, float* fin) {
  using F = FmtT<FMT>;
  constexpr int RB = C::rb;
  const GemvPlan g = make_plan_nrpp(R, K, F::kElems, C::nr, C::pp, C::ks);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int rs = wave / C::ks, sg = wave % C::ks;
  float acc[C::nr];
#pragma unroll
  for (int i = 0; i < C::nr; ++i) acc[i] = 0.f;
#pragma unroll
  for (int q = 0; q < C::pp; ++q) {
    const int pass = plan_pass(g, sg, 0, q);
    if (!pass_valid(g, sg, pass)) continue;
    const int c = pass * kPassChunks + lane;
    if (c < g.nchunks) {
      XPrep<FMT> xp;
      read_prep<FMT>(prep + c * F::kStride, xp);
      if constexpr (kGroupScaled<FMT>) {
        const float bias = chunk_bias<FMT>(xp);
        GroupScales<FMT, C::nr> gs;
#pragma unroll
        for (int j = 0; j < static_cast<int>(sizeof(gs.w) / 4); ++j) gs.w[j] = b.s[q * C::nr + j];
#pragma unroll
        for (int i = 0; i < C::nr; ++i)
          acc[i] = fmaf(gs.scale(i), chunk_dot<FMT>(b.w[i * C::pp + q], xp, bias), acc[i]);
      } else {
#pragma unroll
        for (int i = 0; i < C::nr; ++i) acc[i] = chunk_dot<FMT>(b.w[i * C::pp + q], xp, acc[i]);
      }
    }
  }
  constexpr int L2 = log2i<C::nr>();
  const float s = reduce_rows<C::nr>(acc);
  if ((lane & ((kWave >> L2) - 1)) == 0) part[sg * RB + rs * C::nr + (lane >> (6 - L2))] = s;
  lds_barrier();
  if (threadIdx.x < RB) {
    float v = part[threadIdx.x];
#pragma unroll
    for (int s2 = 1; s2 < C::ks; ++s2) v += part[s2 * RB + threadIdx.x];
    fin[threadIdx.x] = v;
  }
  lds_barrier();
  (void)tile;
}

// Activations of a phase: fp32 vector (coherent loads), optional RMSNorm,
// converted once per workgroup into the GEMV's prepared LDS form.
template <int FMT, bool NORM>
__device__ __forceinline__ void prep_phase(const float* x, const uint16_t* norm_w, float eps, int K, uint32_t* prep,
                                           float* red) {
  using F = FmtT<FMT>;
  constexpr int UPC = F::kElems / 8;
  constexpr int MAXU = 2;  // K <= 4096 for normed phases
  const int nunits = K / 8;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  float inv = 1.f;
  if constexpr (NORM) {
    float v[MAXU][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < MAXU; ++k) {
      const int u = tid + k * kBlock;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[k][e] = u < nunits ? coh_ld(x + 8 * u + e) : 0.f;
        ss += v[k][e] * v[k][e];
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    lds_barrier();
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) ss += red[w];
    inv = 1.f / sqrtf(ss / static_cast<float>(K) + eps);
#pragma unroll
    for (int k = 0; k < MAXU; ++k) {
      const int u = tid + k * kBlock;
      const bool ok = u < nunits;
      const int uu = ok ? u : nunits - 1;
      const u32x4 nw = *reinterpret_cast<const u32x4*>(norm_w + 8 * uu);
      const uint32_t nd[4] = {nw.x, nw.y, nw.z, nw.w};
      float vv[8];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const f16x2 h = as_h2(nd[e2]);
        vv[2 * e2] = (inv * v[k][2 * e2]) * static_cast<float>(h.x);
        vv[2 * e2 + 1] = (inv * v[k][2 * e2 + 1]) * static_cast<float>(h.y);
      }
      uint32_t* dst = prep + (uu / UPC) * F::kStride;
      float cpart = 0.f;
      if (ok) cpart = prep_unit<FMT>(vv, dst, u % UPC);
      if constexpr (UPC > 1) {
        cpart = group_sum<UPC>(cpart);
        if (ok && u % UPC == 0) store_bias<FMT>(dst, cpart);
      }
    }
  } else {
    for (int u0 = 0; u0 < nunits; u0 += kBlock) {
      const int u = u0 + tid;
      const bool ok = u < nunits;
      float vv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) vv[e] = ok ? coh_ld(x + 8 * u + e) : 0.f;
      uint32_t* dst = prep + ((ok ? u : 0) / UPC) * F::kStride;
      float cpart = 0.f;
      if (ok) cpart = prep_unit<FMT>(vv, dst, u % UPC);
      if constexpr (UPC > 1) {
        cpart = group_sum<UPC>(cpart);
        if (ok && u % UPC == 0) store_bias<FMT>(dst, cpart);
      }
    }
  }
  lds_barrier();
}

// Order-preserving 64-bit key of (logit, index): larger logit wins, then the
// lower index (std::max_element's first maximum).
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<uint64_t>(u) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(idx));
}

enum FusedEpi { FE_QKV = 0, FE_RESID = 1, FE_SWIGLU = 2, FE_LOGITS = 3 };

// Epilogue of one tile: threads t < RB own row tile*RB + t (8-row groups are
// whole inside a tile, so RoPE and SwiGLU partners are in fin).
template <int EPI, int RB>
__device__ __forceinline__ void tile_epilogue(const FusedParams& P, const cpi_fused_layer& L, int R, int tile,
                                              const float* fin, int pos, uint64_t& best) {
  const int t = threadIdx.x;
  if (t >= RB) return;
  const int row = tile * RB + t;
  if (row >= R) return;
  const float acc = fin[t];
  if constexpr (EPI == FE_RESID) {
    coh_st(P.x + row, coh_ld(P.x + row) + acc);
  } else if constexpr (EPI == FE_SWIGLU) {
    const int r = row % kTileRows;
    if (r < 4) {
      const float u = fin[t + 4];
      coh_st(P.ff + (row / kTileRows) * 4 + r, (acc / (1.f + expf(-acc))) * u);
    }
  } else if constexpr (EPI == FE_LOGITS) {
    coh_st(P.logits + row, acc);
    const uint64_t k = argmax_key(acc, row);
    best = k > best ? k : best;
  } else {
    // QKV rows in cpi_hip_qkv_row_order: tile T of 8 rows holds rotary pairs
    // (d, d + hd/2) for 4 consecutive d; rows r, r + 1 (r even) are adjacent
    // dims, stored together as one 32-bit coherent word in the fp16 cache.
    if (t & 1) return;
    const int T = row / kTileRows, r = row % kTileRows;
    const int hd = P.hd, half = hd >> 1, tph = hd / kTileRows;
    const int q_tiles = P.nh * tph, k_tiles = P.nkv * tph;
    const int kvdim = P.nkv * hd;
    const float a0 = fin[t], a1 = fin[t + 1];
    if (T < q_tiles + k_tiles) {
      const bool is_q = T < q_tiles;
      const int u = is_q ? T : T - q_tiles;
      const int head = u / tph;
      const int dd = 4 * (u % tph) + (r & 3);
      const float o0 = fin[t ^ 4], o1 = fin[(t + 1) ^ 4];
      const float* cs = P.rope_cos + static_cast<size_t>(pos) * half + dd;
      const float* sn = P.rope_sin + static_cast<size_t>(pos) * half + dd;
      float v0, v1;
      int d;
      if (r < 4) {
        v0 = a0 * cs[0] - o0 * sn[0];
        v1 = a1 * cs[1] - o1 * sn[1];
        d = dd;
      } else {
        v0 = o0 * sn[0] + a0 * cs[0];
        v1 = o1 * sn[1] + a1 * cs[1];
        d = dd + half;
      }
      if (is_q) {
        coh_st(P.q + head * hd + d, v0);
        coh_st(P.q + head * hd + d + 1, v1);
      } else if (pos < P.max_ctx) {
        uint16_t* kc = L.k_cache + static_cast<size_t>(pos) * kvdim + head * hd + d;
        coh_st_u32(reinterpret_cast<uint32_t*>(kc), static_cast<uint32_t>(f2h(v0)) | (static_cast<uint32_t>(f2h(v1)) << 16));
      }
    } else {
      const int vr = (T - q_tiles - k_tiles) * kTileRows + r;
      if (pos < P.max_ctx && vr < kvdim) {
        uint16_t* vc = L.v_cache + static_cast<size_t>(pos) * kvdim + vr;
        coh_st_u32(reinterpret_cast<uint32_t*>(vc), static_cast<uint32_t>(f2h(a0)) | (static_cast<uint32_t>(f2h(a1)) << 16));
      }
    }
  }
}

// One GEMV phase: the first tile's loads are already in `wb` (issued before
// the barrier) when blockIdx.x < tiles.
template <int FMT, class C, int EPI, bool NORM>
__device__ __forceinline__ void gemv_phase(const FusedParams& P, const cpi_fused_layer& L, const uint8_t* W,
                                           const uint16_t* S, int R, int K, const float* x, const uint16_t* norm_w,
                                           int pos, WBuf& wb, uint32_t* prep, float* part, float* fin, float* red,
                                           uint64_t& best) {
  constexpr int RB = C::rb;
  const int tiles = (R + RB - 1) / RB;
  if (static_cast<int>(blockIdx.x) >= tiles) return;
  prep_phase<FMT, NORM>(x, norm_w, P.eps, K, prep, red);
  for (int tile = blockIdx.x; tile < tiles;) {
    tile_compute<FMT, C>(R, K, tile, wb, prep, part, fin);
    const int next = tile + gridDim.x;
    if (next < tiles) tile_issue<FMT, C>(W, S, R, K, next, wb);
    tile_epilogue<EPI, RB>(P, L, R, tile, fin, pos, best);
    tile = next;
  }
}

template <int FMT, class C>
__device__ __forceinline__ void prefetch_first(const uint8_t* W, const uint16_t* S, int R, int K, WBuf& wb) {
  constexpr int RB = C::rb;
  if (static_cast<int>(blockIdx.x) < (R + RB - 1) / RB) tile_issue<FMT, C>(W, S, R, K, blockIdx.x, wb);
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
constexpr int kFusedPrepWords = (12288 / 32) * FmtT<CPI_W_I4G32B>::kStride;  // largest prepared vector
static_assert(kFusedPrepWords >= (4096 / 8) * FmtT<CPI_W_F16>::kStride, "lm_head prep fits");

template <int HD, int GQ>
__global__ void __launch_bounds__(kBlock, 2) decode_fused_kernel(FusedParams P) {
  __shared__ __align__(16) uint32_t prep[kFusedPrepWords];
  __shared__ float part[kWavesPerBlock * 32];
  __shared__ float fin[32];
  __shared__ float red[kWavesPerBlock];
  __shared__ uint64_t wbest[kWavesPerBlock];

  const int H = P.H, I = P.I;
  const int qkv_rows = (P.nh + 2 * P.nkv) * P.hd;
  const int qdim = P.nh * P.hd;
  uint32_t target = 0;
  if (threadIdx.x == 0) target = coh_ld_u32(&P.sync[kSyncBase]);
  const int token = *P.token;
  const int pos = *P.pos;
  uint64_t best = 0;
  bool live = true;
  WBuf wb;

  // ---- embedding row -> x
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < H; i += gridDim.x * kBlock)
    coh_st(P.x + i, h2f(P.emb[static_cast<size_t>(token) * H + i]));
  barrier_arrive(P, target, live);
  {
    const cpi_fused_layer& L0 = P.layers[0];
    prefetch_first<CPI_W_I4G32B, CfgQKV>(static_cast<const uint8_t*>(L0.wqkv), static_cast<const uint16_t*>(L0.sqkv),
                                        qkv_rows, H, wb);
  }
  barrier_wait(P, target, live);

  AttnParams ap{};
  ap.q = P.q;
  ap.out = P.att;
  ap.position = P.pos;
  ap.nh = P.nh;
  ap.nkv = P.nkv;
  ap.max_ctx = P.max_ctx;
  ap.window = P.window;
  ap.nsplit = P.nsplit;
  ap.scale = P.attn_scale;
  ap.scratch = P.attn_scratch;

  for (int l = 0; l < P.nlayers; ++l) {
    const cpi_fused_layer& L = P.layers[l];
    // QKV + RMSNorm + RoPE + KV store
    gemv_phase<CPI_W_I4G32B, CfgQKV, FE_QKV, true>(P, L, static_cast<const uint8_t*>(L.wqkv),
                                                  static_cast<const uint16_t*>(L.sqkv), qkv_rows, H, P.x,
                                                  L.norm_att, pos, wb, prep, part, fin, red, best);
    barrier_arrive(P, target, live);
    barrier_wait(P, target, live);
    // attention: work items (kv head, split)
    ap.k = L.k_cache;
    ap.v = L.v_cache;
    for (int it = blockIdx.x; it < P.nkv * P.nsplit; it += gridDim.x) {
      __syncthreads();  // LDS of the previous item is free
      attn_body<HD, GQ, true, true, true>(ap, it % P.nkv, it / P.nkv);
    }
    barrier_arrive(P, target, live);
    prefetch_first<CPI_W_I4G32B, CfgO>(static_cast<const uint8_t*>(L.wo), static_cast<const uint16_t*>(L.so), H, qdim,
                                      wb);
    barrier_wait(P, target, live);
    // o_proj + residual
    gemv_phase<CPI_W_I4G32B, CfgO, FE_RESID, false>(P, L, static_cast<const uint8_t*>(L.wo),
                                                   static_cast<const uint16_t*>(L.so), H, qdim, P.att, nullptr, pos,
                                                   wb, prep, part, fin, red, best);
    barrier_arrive(P, target, live);
    prefetch_first<CPI_W_I4G32B, CfgW13>(static_cast<const uint8_t*>(L.w13), static_cast<const uint16_t*>(L.s13),
                                        2 * I, H, wb);
    barrier_wait(P, target, live);
    // w1|w3 + RMSNorm + SwiGLU
    gemv_phase<CPI_W_I4G32B, CfgW13, FE_SWIGLU, true>(P, L, static_cast<const uint8_t*>(L.w13),
                                                     static_cast<const uint16_t*>(L.s13), 2 * I, H, P.x,
                                                     L.norm_ffn, pos, wb, prep, part, fin, red, best);
    barrier_arrive(P, target, live);
    prefetch_first<CPI_W_I4G32B, CfgW2>(static_cast<const uint8_t*>(L.w2), static_cast<const uint16_t*>(L.s2), H, I,
                                       wb);
    barrier_wait(P, target, live);
    // w2 + residual
    gemv_phase<CPI_W_I4G32B, CfgW2, FE_RESID, false>(P, L, static_cast<const uint8_t*>(L.w2),
                                                    static_cast<const uint16_t*>(L.s2), H, I, P.ff, nullptr, pos,
                                                    wb, prep, part, fin, red, best);
    barrier_arrive(P, target, live);
    if (l + 1 < P.nlayers) {
      const cpi_fused_layer& N = P.layers[l + 1];
      prefetch_first<CPI_W_I4G32B, CfgQKV>(static_cast<const uint8_t*>(N.wqkv), static_cast<const uint16_t*>(N.sqkv),
                                          qkv_rows, H, wb);
    } else {
      prefetch_first<CPI_W_F16, CfgLM>(reinterpret_cast<const uint8_t*>(P.lm_w), nullptr, P.V, H, wb);
    }
    barrier_wait(P, target, live);
  }

  // ---- final norm + lm_head + argmax
  gemv_phase<CPI_W_F16, CfgLM, FE_LOGITS, true>(P, P.layers[0], reinterpret_cast<const uint8_t*>(P.lm_w), nullptr,
                                                 P.V, H, P.x, P.norm_out, pos, wb, prep, part, fin, red, best);
  // workgroup maximum, then one device-wide atomic max
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const uint64_t o = __shfl_xor(best, m, kWave);
    best = o > best ? o : best;
  }
  if (lane == 0) wbest[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = wbest[0];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) b = wbest[w] > b ? wbest[w] : b;
    if (b != 0)
      __hip_atomic_fetch_max(reinterpret_cast<uint64_t*>(P.sync + kSyncArgmax), b, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  barrier_arrive(P, target, live);
  barrier_wait(P, target, live);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    uint64_t* kp = reinterpret_cast<uint64_t*>(P.sync + kSyncArgmax);
    const uint64_t k = __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int idx = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(k & 0xFFFFFFFFu));
    const int tok = (k == 0 || idx < 0 || idx >= P.V) ? 0 : idx;
    __hip_atomic_store(kp, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int st = *P.step;
    P.ring[st % P.ring_len] = tok;
    *P.step = st + 1;
    *P.token = tok;
    *P.pos = pos + 1;
    coh_st_u32(&P.sync[kSyncBase], target);
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
template <int FMT>
constexpr int np_of(int K) {
  return (K / FmtT<FMT>::kElems + kPassChunks - 1) / kPassChunks;
}

bool fused_supported(const cpi_fused_decode_desc& d, const char** why) {
  auto no = [&](const char* m) {
    *why = m;
    return false;
  };
  if (d.head_dim != 64 && d.head_dim != 128) return no("head_dim must be 64 or 128");
  if (d.num_kv_heads <= 0 || d.num_heads % d.num_kv_heads != 0) return no("bad head counts");
  const int G = d.num_heads / d.num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return no("GQA group must be 1, 2, 4 or 8");
  const int qdim = d.num_heads * d.head_dim;
  if (d.hidden % 32 || d.intermediate % 32 || qdim % 32) return no("dims must be multiples of 32");
  if (np_of<CPI_W_I4G32B>(d.hidden) > CfgQKV::pp * CfgQKV::ks || np_of<CPI_W_I4G32B>(d.hidden) > CfgW13::pp * CfgW13::ks)
    return no("hidden too large for the fused tiles");
  if (np_of<CPI_W_I4G32B>(qdim) > CfgO::pp * CfgO::ks) return no("q dim too large for the fused tiles");
  if (np_of<CPI_W_I4G32B>(d.intermediate) > CfgW2::pp * CfgW2::ks) return no("intermediate too large");
  if (np_of<CPI_W_F16>(d.hidden) > CfgLM::pp * CfgLM::ks) return no("hidden too large for the lm_head tiles");
  if (d.hidden > 4096) return no("hidden > 4096");
  if (d.intermediate / 32 * FmtT<CPI_W_I4G32B>::kStride > kFusedPrepWords) return no("intermediate too large");
  if (d.intermediate % 4 != 0) return no("intermediate % 4");
  return true;
}

template <int HD, int GQ>
hipError_t fused_launch_t(const FusedParams& P, int wgs, hipStream_t s) {
  hipLaunchKernelGGL((decode_fused_kernel<HD, GQ>), dim3(wgs), dim3(kBlock), 0, s, P);
  return hipGetLastError();
}

template <int HD, int GQ>
int fused_max_wgs_t() {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&decode_fused_kernel<HD, GQ>),
                                                   kBlock, 0) != hipSuccess)
    return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return per_cu * cus;
}

#define CPI_FUSED_DISPATCH(FN, ...)                                   \
  switch (hd * 16 + gq) {                                             \
    case 64 * 16 + 1: return FN<64, 1>(__VA_ARGS__);                  \
    case 64 * 16 + 2: return FN<64, 2>(__VA_ARGS__);                  \
    case 64 * 16 + 4: return FN<64, 4>(__VA_ARGS__);                  \
    case 64 * 16 + 8: return FN<64, 8>(__VA_ARGS__);                  \
    case 128 * 16 + 1: return FN<128, 1>(__VA_ARGS__);                \
    case 128 * 16 + 2: return FN<128, 2>(__VA_ARGS__);                \
    case 128 * 16 + 4: return FN<128, 4>(__VA_ARGS__);                \
    case 128 * 16 + 8: return FN<128, 8>(__VA_ARGS__);                \
  }

int fused_max_wgs(int hd, int gq) {
  CPI_FUSED_DISPATCH(fused_max_wgs_t)
  return 0;
}

hipError_t fused_launch(const FusedParams& P, int hd, int gq, int wgs, hipStream_t s) {
  CPI_FUSED_DISPATCH(fused_launch_t, P, wgs, s)
  return hipErrorInvalidValue;
}

}  // namespace cpi

// Decode kernels of the routed-expert MoE layer for gfx950 (wave64).
//
//   k_router   router GEMV over bf16 weights, then (last block to finish)
//              softmax, top-k and renormalisation for every token; one extra
//              block evaluates the shared expert's sigmoid gate.
//   k_gateup   gate and up Q4/G32 GEMV of every (token, slot) pair plus the
//              shared-expert pair, SwiGLU fused in the epilogue.
//   k_down     down Q4/G32 GEMV of every slot of a token for a tile of output
//              rows, and the router-score combine with the shared term.
//
// All three are HBM-bandwidth kernels: one 16-byte load per lane covers one
// 32-input group of one row (4 packed words); scales and biases are 2-byte
// loads that coalesce into one 128-byte line per row; activations sit in
// registers (gate/up, router) or LDS (down); row sums use DPP.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <type_traits>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kBlock = 256;

template <class A>
constexpr bool is_bf16() {
  return std::is_same<A, ActBF16>::value;
}

// Activation chunk of one group held in registers by one lane.
template <class A>
struct GroupAct;

template <>
struct GroupAct<ActBF16> {
  uint32_t xp[16];  // (x_{8i+n}, x_{8i+n+4}) pairs
  float sum;        // sum of the 32 inputs
  float sum128;     // 128 * sum
  __device__ __forceinline__ void load(const void* base, size_t elem) {
    const uint4* v = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem);
    uint32_t raw[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 r = v[q];
      raw[4 * q + 0] = r.x; raw[4 * q + 1] = r.y; raw[4 * q + 2] = r.z; raw[4 * q + 3] = r.w;
    }
    pair_activations(raw, xp);
    sum = bf16_pair_sum(raw);
    sum128 = 128.0f * sum;
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int m = 0; m < 16; ++m) xp[m] = 0;
    sum = 0.0f;
    sum128 = 0.0f;
  }
  // scale * sum(q x) + bias * sum(x)
  __device__ __forceinline__ float apply(const uint4 w, float s, float b) const {
    const float d = q4_dot_bf16(w, xp);
    return fmaf(s, d - sum128, b * sum);
  }
};

template <>
struct GroupAct<ActF32> {
  float x[32];
  float sum;
  __device__ __forceinline__ void load(const void* base, size_t elem) {
    const float4* v = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 r = v[q];
      x[4 * q + 0] = r.x; x[4 * q + 1] = r.y; x[4 * q + 2] = r.z; x[4 * q + 3] = r.w;
      s += r.x + r.y + r.z + r.w;
    }
    sum = s;
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int m = 0; m < 32; ++m) x[m] = 0.0f;
    sum = 0.0f;
  }
  __device__ __forceinline__ float apply(const uint4 w, float s, float b) const {
    const float d = q4_dot_f32(w, x);
    return fmaf(s, d, b * sum);
  }
};

__device__ __forceinline__ void flag(uint32_t* status, uint32_t bits) {
  if (status != nullptr) atomicOr(status, bits);
}

// ------------------------------------------------------------- gate/up ----

template <class A, int LPR, int GI, int U>
__global__ __launch_bounds__(kBlock) void k_gateup(GateUpLaunch p) {
  constexpr int RPI = 64 / LPR;
  constexpr int RPW = RPI * U;
  constexpr int RPB = RPW * (kBlock / 64);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t lr = lane % LPR;
  const uint32_t rw = lane / LPR;

  const uint32_t pair = blockIdx.y;
  const uint32_t routed_pairs = p.tokens * p.slots;
  const bool shared_pair = pair >= routed_pairs;
  const uint32_t t = shared_pair ? pair - routed_pairs : pair / p.slots;
  const uint32_t j = shared_pair ? p.slots : pair % p.slots;
  const uint32_t S = p.slots + p.has_shared;
  const uint32_t H = p.hidden, I = p.inter, G = H / kGroup;

  ProjPtrs gp{}, upp{};
  bool ok = true;
  if (shared_pair) {
    gp = p.shared_gate;
    upp = p.shared_up;
  } else {
    const uint32_t word = p.routes[t * p.slots + j];
    ok = resolve_proj(word, p.slot_table, p.experts, p.pool, p.gate, 0, I, H, gp, &p.stream) &&
         resolve_proj(word, p.slot_table, p.experts, p.pool, p.up, 1, I, H, upp, &p.stream);
  }
  const uint32_t row_base = blockIdx.x * RPB + wave * RPW + rw;
  const size_t act_base = (static_cast<size_t>(t) * S + j) * I;
  if (!ok) {
    if (lr == LPR - 1) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t row = row_base + u * RPI;
        if (row < I) A::store(p.act, act_base + row, 0.0f);
      }
    }
    if (threadIdx.x == 0 && blockIdx.x == 0) flag(p.status, 1u);
    return;
  }

  // Weight loads first so they are in flight while the activations arrive.
  uint4 wg[U][GI], wu[U][GI];
  uint32_t sg[U][GI], bg[U][GI], su[U][GI], bu[U][GI];
  const size_t row_words = H / 8;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t row = row_base + u * RPI;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      const uint32_t g = lr + it * LPR;
      if (row < I && g < G) {
        const size_t wo = row * row_words + g * kWordsPerGroup;
        const size_t mo = static_cast<size_t>(row) * G + g;
        wg[u][it] = *reinterpret_cast<const uint4*>(gp.w + wo);
        wu[u][it] = *reinterpret_cast<const uint4*>(upp.w + wo);
        sg[u][it] = gp.s[mo];
        bg[u][it] = gp.b[mo];
        su[u][it] = upp.s[mo];
        bu[u][it] = upp.b[mo];
      } else {
        wg[u][it] = wu[u][it] = make_uint4(0, 0, 0, 0);
        sg[u][it] = bg[u][it] = su[u][it] = bu[u][it] = 0;
      }
    }
  }
  GroupAct<A> xa[GI];
#pragma unroll
  for (int it = 0; it < GI; ++it) {
    const uint32_t g = lr + it * LPR;
    if (g < G) {
      xa[it].load(p.x, static_cast<size_t>(t) * H + g * kGroup);
    } else {
      xa[it].zero();
    }
  }

#pragma unroll
  for (int u = 0; u < U; ++u) {
    float ag = 0.0f, au = 0.0f;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
      ag += xa[it].apply(wg[u][it], bf16_to_f32(sg[u][it]), bf16_to_f32(bg[u][it]));
      au += xa[it].apply(wu[u][it], bf16_to_f32(su[u][it]), bf16_to_f32(bu[u][it]));
    }
    ag = group_sum<LPR>(ag);
    au = group_sum<LPR>(au);
    const uint32_t row = row_base + u * RPI;
    if (lr == LPR - 1 && row < I) {
      const float gv = A::round(ag);
      const float uv = A::round(au);
      A::store(p.act, act_base + row, swiglu_act<A>(gv, uv));
      if (!shared_pair) {
        const size_t o = (static_cast<size_t>(t) * p.slots + j) * I + row;
        if (p.gate_out != nullptr) A::store(p.gate_out, o, gv);
        if (p.up_out != nullptr) A::store(p.up_out, o, uv);
      }
    }
  }
}

// ----------------------------------------------------------------- down ---

constexpr int kDownMaxSlots = 12;  // MAX_TOP_K (10) + shared, rounded up
constexpr int kDownQuads = 2;      // row groups of 64/LPR rows per block
constexpr int kDownMaxUnits = (kDownMaxSlots * kDownQuads + 3) / 4;

template <class A>
constexpr int lds_group_words() {
  return is_bf16<A>() ? 20 : 36;  // 16 or 32 payload words + 4 words of bank padding
}

template <class A, int LPR>
__global__ __launch_bounds__(kBlock) void k_down(DownLaunch p) {
  constexpr int RPI = 64 / LPR;
  constexpr int RB = RPI * kDownQuads;
  constexpr int GW = lds_group_words<A>();
  extern __shared__ uint4 lds_raw[];
  uint32_t* lds_act = reinterpret_cast<uint32_t*>(lds_raw);

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t lr = lane % LPR;
  const uint32_t rw = lane / LPR;
  const uint32_t t = blockIdx.y;
  const uint32_t K = p.slots;
  const uint32_t S = K + p.has_shared;
  const uint32_t H = p.hidden, I = p.inter, G = I / kGroup;
  const uint32_t row0 = blockIdx.x * RB;
  float* lds_sum = reinterpret_cast<float*>(lds_act + S * G * GW);
  float* lds_part = lds_sum + S * G;

  // 1. resolve this wave's units and issue their weight loads
  uint4 w[kDownMaxUnits];
  uint32_t sc[kDownMaxUnits], bi[kDownMaxUnits];
  bool live[kDownMaxUnits];
  const size_t row_words = I / 8;
#pragma unroll
  for (int i = 0; i < kDownMaxUnits; ++i) {
    const uint32_t unit = wave + 4 * i;
    const uint32_t slot = unit / kDownQuads;
    const uint32_t quad = unit % kDownQuads;
    const uint32_t row = row0 + quad * RPI + rw;
    live[i] = unit < S * kDownQuads;
    ProjPtrs dp{};
    bool ok = false;
    if (live[i]) {
      if (slot < K) {
        ok = resolve_proj(p.routes[t * K + slot], p.slot_table, p.experts, p.pool, p.down, 2, H, I, dp,
                          &p.stream);
        if (!ok && threadIdx.x % 64 == 0 && blockIdx.x == 0) flag(p.status, 1u);
      } else {
        dp = p.shared_down;
        ok = true;
      }
    }
    if (ok && row < H && lr < G) {
      w[i] = *reinterpret_cast<const uint4*>(dp.w + row * row_words + lr * kWordsPerGroup);
      sc[i] = dp.s[static_cast<size_t>(row) * G + lr];
      bi[i] = dp.b[static_cast<size_t>(row) * G + lr];
    } else {
      w[i] = make_uint4(0, 0, 0, 0);
      sc[i] = bi[i] = 0;
    }
  }

  // 2. stage the token's activations (all slots) into LDS in dot order
  for (uint32_t item = threadIdx.x; item < S * G; item += kBlock) {
    const uint32_t slot = item / G, g = item % G;
    const size_t elem = (static_cast<size_t>(t) * S + slot) * I + g * kGroup;
    uint32_t* dst = lds_act + item * GW;
    if constexpr (is_bf16<A>()) {
      const uint4* v = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.act) + elem);
      uint32_t raw[16], xp[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 r = v[q];
        raw[4 * q + 0] = r.x; raw[4 * q + 1] = r.y; raw[4 * q + 2] = r.z; raw[4 * q + 3] = r.w;
      }
      pair_activations(raw, xp);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        reinterpret_cast<uint4*>(dst)[q] = make_uint4(xp[4 * q], xp[4 * q + 1], xp[4 * q + 2], xp[4 * q + 3]);
      lds_sum[item] = bf16_pair_sum(raw);
    } else {
      const float4* v = reinterpret_cast<const float4*>(static_cast<const float*>(p.act) + elem);
      float s = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float4 r = v[q];
        reinterpret_cast<float4*>(dst)[q] = r;
        s += r.x + r.y + r.z + r.w;
      }
      lds_sum[item] = s;
    }
  }
  __syncthreads();

  // 3. dot products, row sums, partials to LDS
#pragma unroll
  for (int i = 0; i < kDownMaxUnits; ++i) {
    const uint32_t unit = wave + 4 * i;
    if (unit >= S * kDownQuads) break;  // wave-uniform
    const uint32_t slot = unit / kDownQuads;
    const uint32_t quad = unit % kDownQuads;
    float v = 0.0f;
    if (lr < G) {
      const uint32_t item = slot * G + lr;
      const uint32_t* src = lds_act + item * GW;
      const float s = bf16_to_f32(sc[i]), b = bf16_to_f32(bi[i]);
      const float xs = lds_sum[item];
      if constexpr (is_bf16<A>()) {
        uint32_t xp[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint4 r = reinterpret_cast<const uint4*>(src)[q];
          xp[4 * q] = r.x; xp[4 * q + 1] = r.y; xp[4 * q + 2] = r.z; xp[4 * q + 3] = r.w;
        }
        v = fmaf(s, q4_dot_bf16(w[i], xp) - 128.0f * xs, b * xs);
      } else {
        float x[32];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float4 r = reinterpret_cast<const float4*>(src)[q];
          x[4 * q] = r.x; x[4 * q + 1] = r.y; x[4 * q + 2] = r.z; x[4 * q + 3] = r.w;
        }
        v = fmaf(s, q4_dot_f32(w[i], x), b * xs);
      }
    }
    v = group_sum<LPR>(v);
    if (lr == LPR - 1) lds_part[slot * RB + quad * RPI + rw] = v;
  }
  __syncthreads();

  // 4. epilogue
  if (p.scores != nullptr) {
    for (uint32_t r = threadIdx.x; r < RB; r += kBlock) {
      const uint32_t row = row0 + r;
      if (row >= H) continue;
      float combined = 0.0f;
      for (uint32_t k = 0; k < K; ++k) {
        const float d = A::round(lds_part[k * RB + r]);
        const float sc_k = load_any(p.scores, static_cast<size_t>(t) * K + k, p.score_dtype);
        combined = __fadd_rn(combined, __fmul_rn(d, sc_k));
      }
      float y = A::round(combined);
      const size_t o = static_cast<size_t>(t) * H + row;
      if (p.has_shared) {
        const float sh = A::round(lds_part[K * RB + r]);
        const float sy = A::round(__fmul_rn(A::load(p.shared_sig, t), sh));
        y = A::round(__fadd_rn(y, sy));
      } else if (p.shared_y != nullptr) {
        y = A::round(__fadd_rn(y, A::load(p.shared_y, o)));
      } else if (p.shared != nullptr) {
        const float comp = A::round(__fmul_rn(A::load(p.shared, o), A::load(p.shared_gate, t)));
        y = A::round(__fadd_rn(y, comp));
      }
      A::store(p.out, o, y);
    }
  } else {
    for (uint32_t idx = threadIdx.x; idx < K * RB; idx += kBlock) {
      const uint32_t k = idx / RB, r = idx % RB;
      const uint32_t row = row0 + r;
      if (row < H) A::store(p.out, (static_cast<size_t>(t) * K + k) * H + row, A::round(lds_part[k * RB + r]));
    }
  }
}

// --------------------------------------------------------------- router ---

constexpr int kRouterRowsPerWave = 2;
constexpr int kRouterRowsPerBlock = kRouterRowsPerWave * (kBlock / 64);
constexpr int kRouterMaxChunks = 16;  // hidden <= 16 * 512 = 8192
constexpr int kMaxExpertsPerLane = 8; // expert_count <= 512

// dot of 8 bf16 weights with 8 activations (one 16-byte chunk)
template <class A>
struct RouterChunk;

template <>
struct RouterChunk<ActBF16> {
  uint4 x;
  __device__ __forceinline__ void load(const void* base, size_t elem) {
    x = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + elem);
  }
  __device__ __forceinline__ void zero() { x = make_uint4(0, 0, 0, 0); }
  __device__ __forceinline__ float dot(const uint4 w, float acc) const {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.x), __builtin_bit_cast(bf16x2, x.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.y), __builtin_bit_cast(bf16x2, x.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.z), __builtin_bit_cast(bf16x2, x.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.w), __builtin_bit_cast(bf16x2, x.w), acc, false);
    return acc;
  }
};

template <>
struct RouterChunk<ActF32> {
  float4 a, b;
  __device__ __forceinline__ void load(const void* base, size_t elem) {
    const float4* v = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
    a = v[0];
    b = v[1];
  }
  __device__ __forceinline__ void zero() { a = b = make_float4(0, 0, 0, 0); }
  __device__ __forceinline__ float dot(const uint4 w, float acc) const {
    acc = fmaf(bf16_to_f32(w.x & 0xffffu), a.x, acc);
    acc = fmaf(bf16_to_f32(w.x >> 16), a.y, acc);
    acc = fmaf(bf16_to_f32(w.y & 0xffffu), a.z, acc);
    acc = fmaf(bf16_to_f32(w.y >> 16), a.w, acc);
    acc = fmaf(bf16_to_f32(w.z & 0xffffu), b.x, acc);
    acc = fmaf(bf16_to_f32(w.z >> 16), b.y, acc);
    acc = fmaf(bf16_to_f32(w.w & 0xffffu), b.z, acc);
    acc = fmaf(bf16_to_f32(w.w >> 16), b.w, acc);
    return acc;
  }
};

// Router rows for a single token, activations in registers.  CH = 16-byte
// chunks per lane per row (hidden / 512, rounded up).
template <class A, int CH>
__device__ void router_rows_one(const RouterLaunch& p, uint32_t row0, uint32_t lane) {
  const uint32_t H = p.hidden;
  RouterChunk<A> xc[CH];
  uint4 w[kRouterRowsPerWave][CH];
#pragma unroll
  for (int r = 0; r < kRouterRowsPerWave; ++r) {
    const uint32_t row = row0 + r;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t e8 = 8 * (lane + 64 * c);
      if (row < p.experts && e8 < H) {
        w[r][c] = *reinterpret_cast<const uint4*>(p.weight + static_cast<size_t>(row) * H + e8);
      } else {
        w[r][c] = make_uint4(0, 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const uint32_t e8 = 8 * (lane + 64 * c);
    if (e8 < H) xc[c].load(p.x, e8); else xc[c].zero();
  }
#pragma unroll
  for (int r = 0; r < kRouterRowsPerWave; ++r) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) acc = xc[c].dot(w[r][c], acc);
    acc = group_sum<64>(acc);
    const uint32_t row = row0 + r;
    if (lane == 63 && row < p.experts) {
      if (p.bias != nullptr) acc += p.bias[row];
      p.logits[row] = A::round(acc);
    }
  }
}

// Router rows for several tokens: weights in registers, activations re-read per token.
template <class A, int CH>
__device__ void router_rows_many(const RouterLaunch& p, uint32_t row0, uint32_t lane) {
  const uint32_t H = p.hidden;
  uint4 w[kRouterRowsPerWave][CH];
#pragma unroll
  for (int r = 0; r < kRouterRowsPerWave; ++r) {
    const uint32_t row = row0 + r;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t e8 = 8 * (lane + 64 * c);
      if (row < p.experts && e8 < H) {
        w[r][c] = *reinterpret_cast<const uint4*>(p.weight + static_cast<size_t>(row) * H + e8);
      } else {
        w[r][c] = make_uint4(0, 0, 0, 0);
      }
    }
  }
  for (uint32_t t = 0; t < p.tokens; ++t) {
    float acc[kRouterRowsPerWave] = {};
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t e8 = 8 * (lane + 64 * c);
      if (e8 < H) {
        RouterChunk<A> xc;
        xc.load(p.x, static_cast<size_t>(t) * H + e8);
#pragma unroll
        for (int r = 0; r < kRouterRowsPerWave; ++r) acc[r] = xc.dot(w[r][c], acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < kRouterRowsPerWave; ++r) {
      const float v = group_sum<64>(acc[r]);
      const uint32_t row = row0 + r;
      if (lane == 63 && row < p.experts) {
        p.logits[static_cast<size_t>(t) * p.experts + row] =
            A::round(p.bias != nullptr ? v + p.bias[row] : v);
      }
    }
  }
}

// Softmax, top-k by (gate desc, index asc), renormalisation: one wave per token.
template <class A>
__device__ void router_select(const RouterLaunch& p, uint32_t t, uint32_t lane) {
  const uint32_t E = p.experts;
  const uint32_t K = p.top_k;
  float l[kMaxExpertsPerLane];
  float lmax = -FLT_MAX;
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t e = lane + 64 * m;
    l[m] = e < E ? p.logits[static_cast<size_t>(t) * E + e] : -FLT_MAX;
    lmax = fmaxf(lmax, l[m]);
  }
  lmax = wave_max_f32(lmax);
  float ex[kMaxExpertsPerLane];
  float local = 0.0f;
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t e = lane + 64 * m;
    ex[m] = e < E ? expf(l[m] - lmax) : 0.0f;
    local += ex[m];
  }
  const float total = wave_sum_all(local);
  uint32_t gbits[kMaxExpertsPerLane];
  bool taken[kMaxExpertsPerLane];
#pragma unroll
  for (int m = 0; m < kMaxExpertsPerLane; ++m) {
    const uint32_t e = lane + 64 * m;
    const float gate = A::round(ex[m] / total);
    if (p.gates != nullptr && e < E) A::store(p.gates, static_cast<size_t>(t) * E + e, gate);
    // gates are >= 0, so their bit patterns order like their values
    gbits[m] = is_bf16<A>() ? f32_to_bf16(gate) : __float_as_uint(gate);
    taken[m] = e >= E;
  }

  // k rounds of a wave-wide max over (gate bits, inverted index) keys; lane k
  // keeps the k-th winner.
  int my_e = 0;
  float my_g = 0.0f;
  float mass = 0.0f;
  for (uint32_t k = 0; k < K; ++k) {
    uint32_t best_key = 0, best_inv = 0;
#pragma unroll
    for (int m = 0; m < kMaxExpertsPerLane; ++m) {
      if (taken[m]) continue;
      const uint32_t e = lane + 64 * m;
      if (is_bf16<A>()) {
        const uint32_t key = (gbits[m] << 16) | (0xffffu - e);
        if (key > best_key) best_key = key;
      } else {
        const uint32_t inv = 0xffffffffu - e;
        if (gbits[m] > best_key || (gbits[m] == best_key && inv > best_inv)) {
          best_key = gbits[m];
          best_inv = inv;
        }
      }
    }
    uint32_t win_e;
    float win_g;
    if (is_bf16<A>()) {
      // every live key has a non-zero inverted index, so 0 means "none left"
      const uint32_t win = wave_max_u32(best_key);
      win_e = 0xffffu - (win & 0xffffu);
      win_g = bf16_to_f32(win >> 16);
    } else {
      const uint32_t top = wave_max_u32(best_key);
      const uint32_t inv = wave_max_u32(best_key == top ? best_inv : 0u);
      win_e = 0xffffffffu - inv;
      win_g = __uint_as_float(top);
    }
    mass += win_g;
    if (lane == k) {
      my_e = static_cast<int>(win_e);
      my_g = win_g;
    }
#pragma unroll
    for (int m = 0; m < kMaxExpertsPerLane; ++m) {
      if (lane + 64 * m == win_e) taken[m] = true;
    }
  }
  // scores / (mass + blend * (selected - mass)), each step rounded
  mass = A::round(mass);
  const float diff = A::round(mass - mass);
  const float normalizer = A::round(mass + A::round(p.blend * diff));
  if (lane < K) {
    p.inds[static_cast<size_t>(t) * K + lane] = my_e;
    A::store(p.scores, static_cast<size_t>(t) * K + lane, A::round(my_g / normalizer));
  }
}

// The shared expert's H -> 1 quantized gate followed by the sigmoid.
template <class A>
__device__ void shared_gate_logit(const RouterLaunch& p, uint32_t lane) {
  const uint32_t H = p.hidden, G = H / kGroup;
  for (uint32_t t = 0; t < p.tokens; ++t) {
    float acc = 0.0f;
    for (uint32_t g = lane; g < G; g += 64) {
      const uint4 w = *reinterpret_cast<const uint4*>(p.seg.w + g * kWordsPerGroup);
      GroupAct<A> xa;
      xa.load(p.x, static_cast<size_t>(t) * H + g * kGroup);
      acc += xa.apply(w, bf16_to_f32(p.seg.s[g]), bf16_to_f32(p.seg.b[g]));
    }
    const float logit = A::round(wave_sum_all(acc));
    if (lane == 0) A::store(p.shared_sig, t, sigmoid_act<A>(logit));
  }
}

template <class A, bool ONE, int CH>
__global__ __launch_bounds__(kBlock) void k_router(RouterLaunch p, uint32_t router_blocks) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  if (blockIdx.x >= router_blocks) {
    if (wave == 0) shared_gate_logit<A>(p, lane);
    return;
  }
  const uint32_t row0 = blockIdx.x * kRouterRowsPerBlock + wave * kRouterRowsPerWave;
  if (ONE) router_rows_one<A, CH>(p, row0, lane); else router_rows_many<A, CH>(p, row0, lane);

  // The last router block to finish runs the selection for every token.
  __shared__ uint32_t last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = atomicAdd(p.counter, 1u) == router_blocks - 1 ? 1u : 0u;
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (uint32_t t = wave; t < p.tokens; t += kBlock / 64) router_select<A>(p, t, lane);
  __syncthreads();
  if (threadIdx.x == 0) atomicExch(p.counter, 0u);
}

// ------------------------------------------------------ weighted combine --

template <class A>
__global__ __launch_bounds__(kBlock) void k_weighted_combine(const void* values, const void* scores, void* out,
                                                             uint32_t tokens, uint32_t slots, uint32_t hidden,
                                                             int score_dtype) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= static_cast<size_t>(tokens) * hidden) return;
  const uint32_t t = static_cast<uint32_t>(i / hidden), h = static_cast<uint32_t>(i % hidden);
  float acc = 0.0f;
  for (uint32_t k = 0; k < slots; ++k) {
    const float v = A::load(values, (static_cast<size_t>(t) * slots + k) * hidden + h);
    acc = __fadd_rn(acc, __fmul_rn(v, load_any(scores, static_cast<size_t>(t) * slots + k, score_dtype)));
  }
  A::store(out, i, A::round(acc));
}

// ------------------------------------------------------------ dispatch ----

uint32_t next_pow2(uint32_t v) {
  uint32_t r = 1;
  while (r < v) r <<= 1;
  return r;
}

template <class A, int LPR, int GI, int U>
hipError_t gateup_go(const GateUpLaunch& p, hipStream_t stream) {
  constexpr int RPB = (64 / LPR) * U * (kBlock / 64);
  const uint32_t pairs = p.tokens * p.slots + (p.has_shared ? p.tokens : 0);
  dim3 grid((p.inter + RPB - 1) / RPB, pairs);
  hipLaunchKernelGGL((k_gateup<A, LPR, GI, U>), grid, dim3(kBlock), 0, stream, p);
  return hipGetLastError();
}

template <class A>
hipError_t gateup_dispatch(const GateUpLaunch& p, hipStream_t stream) {
  const uint32_t G = p.hidden / kGroup;
  const uint32_t lpr = G >= 64 ? 64 : next_pow2(G);
  const uint32_t gi = (G + 63) / 64;
  switch (lpr) {
    case 1: return gateup_go<A, 1, 1, 1>(p, stream);
    case 2: return gateup_go<A, 2, 1, 1>(p, stream);
    case 4: return gateup_go<A, 4, 1, 1>(p, stream);
    case 8: return gateup_go<A, 8, 1, 1>(p, stream);
    case 16: return gateup_go<A, 16, 1, 2>(p, stream);
    case 32: return gateup_go<A, 32, 1, 2>(p, stream);
    default: break;
  }
  if (gi <= 1) return gateup_go<A, 64, 1, 2>(p, stream);
  if (gi <= 2) return gateup_go<A, 64, 2, 2>(p, stream);
  return gateup_go<A, 64, 4, 1>(p, stream);
}

template <class A>
size_t down_lds_bytes(uint32_t slots_total, uint32_t inter, uint32_t lpr) {
  const uint32_t G = inter / kGroup;
  const uint32_t rb = (64 / lpr) * kDownQuads;
  return static_cast<size_t>(slots_total) * G * lds_group_words<A>() * 4 + slots_total * G * 4 +
         static_cast<size_t>(slots_total) * rb * 4;
}

template <class A, int LPR>
hipError_t down_go(const DownLaunch& p, hipStream_t stream) {
  constexpr int RB = (64 / LPR) * kDownQuads;
  const uint32_t S = p.slots + p.has_shared;
  const size_t lds = down_lds_bytes<A>(S, p.inter, LPR);
  static size_t attr_bytes = 64 * 1024;
  if (lds > attr_bytes) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_down<A, LPR>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr_bytes = lds;
  }
  dim3 grid((p.hidden + RB - 1) / RB, p.tokens);
  hipLaunchKernelGGL((k_down<A, LPR>), grid, dim3(kBlock), lds, stream, p);
  return hipGetLastError();
}

template <class A>
hipError_t down_dispatch(const DownLaunch& p, hipStream_t stream) {
  const uint32_t G = p.inter / kGroup;
  switch (next_pow2(G)) {
    case 1: return down_go<A, 1>(p, stream);
    case 2: return down_go<A, 2>(p, stream);
    case 4: return down_go<A, 4>(p, stream);
    case 8: return down_go<A, 8>(p, stream);
    case 16: return down_go<A, 16>(p, stream);
    case 32: return down_go<A, 32>(p, stream);
    default: return down_go<A, 64>(p, stream);
  }
}

}  // namespace

bool gateup_supported(uint32_t hidden) {
  return hidden % kGroup == 0 && hidden > 0 && hidden / kGroup <= 256;
}

bool down_supported(uint32_t inter, uint32_t slots_total, int act_dtype) {
  if (inter % kGroup != 0 || inter == 0 || inter / kGroup > 64) return false;
  if (slots_total > static_cast<uint32_t>(kDownMaxSlots) || slots_total == 0) return false;
  const uint32_t lpr = next_pow2(inter / kGroup);
  const size_t lds = act_dtype == 0 ? down_lds_bytes<ActBF16>(slots_total, inter, lpr)
                                    : down_lds_bytes<ActF32>(slots_total, inter, lpr);
  return lds <= 160 * 1024;
}

hipError_t launch_gateup(const GateUpLaunch& p, hipStream_t stream) {
  timing_begin("gateup", stream);
  hipError_t e = p.act_dtype == 0 ? gateup_dispatch<ActBF16>(p, stream) : gateup_dispatch<ActF32>(p, stream);
  timing_end("gateup", stream);
  return e;
}

hipError_t launch_down(const DownLaunch& p, hipStream_t stream) {
  timing_begin("down", stream);
  hipError_t e = p.act_dtype == 0 ? down_dispatch<ActBF16>(p, stream) : down_dispatch<ActF32>(p, stream);
  timing_end("down", stream);
  return e;
}

template <class A, bool ONE>
void router_go(const RouterLaunch& p, uint32_t blocks, uint32_t router_blocks, hipStream_t stream) {
  const uint32_t chunks = (p.hidden / 8 + 63) / 64;
  if (chunks <= 1) hipLaunchKernelGGL((k_router<A, ONE, 1>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else if (chunks <= 2) hipLaunchKernelGGL((k_router<A, ONE, 2>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else if (chunks <= 4) hipLaunchKernelGGL((k_router<A, ONE, 4>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else if (chunks <= 8) hipLaunchKernelGGL((k_router<A, ONE, 8>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
  else hipLaunchKernelGGL((k_router<A, ONE, 16>), dim3(blocks), dim3(kBlock), 0, stream, p, router_blocks);
}

hipError_t launch_router(const RouterLaunch& p, hipStream_t stream) {
  const uint32_t router_blocks = (p.experts + kRouterRowsPerBlock - 1) / kRouterRowsPerBlock;
  const uint32_t blocks = router_blocks + (p.seg.w != nullptr ? 1 : 0);
  timing_begin("router", stream);
  const bool one = p.tokens == 1;
  if (p.act_dtype == 0) {
    if (one) router_go<ActBF16, true>(p, blocks, router_blocks, stream);
    else router_go<ActBF16, false>(p, blocks, router_blocks, stream);
  } else {
    if (one) router_go<ActF32, true>(p, blocks, router_blocks, stream);
    else router_go<ActF32, false>(p, blocks, router_blocks, stream);
  }
  hipError_t e = hipGetLastError();
  timing_end("router", stream);
  return e;
}

hipError_t launch_weighted_combine(const void* values, const void* scores, void* out, uint32_t tokens,
                                   uint32_t slots, uint32_t hidden, int act_dtype, int score_dtype,
                                   hipStream_t stream) {
  const size_t n = static_cast<size_t>(tokens) * hidden;
  const uint32_t blocks = static_cast<uint32_t>((n + kBlock - 1) / kBlock);
  timing_begin("combine", stream);
  if (act_dtype == 0) {
    hipLaunchKernelGGL(k_weighted_combine<ActBF16>, dim3(blocks), dim3(kBlock), 0, stream, values, scores, out,
                       tokens, slots, hidden, score_dtype);
  } else {
    hipLaunchKernelGGL(k_weighted_combine<ActF32>, dim3(blocks), dim3(kBlock), 0, stream, values, scores, out,
                       tokens, slots, hidden, score_dtype);
  }
  hipError_t e = hipGetLastError();
  timing_end("combine", stream);
  return e;
}

}  // namespace vm

// Decoder glue around the MoE call (gfx950): the hyper-connection that makes
// the MoE branch's input from the residual streams.  The injection of the
// branch output back into the streams runs in the MoE's own final epilogue
// (k_down, k_grouped_combine), so it costs no launch.
//
// The hidden state of a token holds hc streams of H values (n = hc * H).
// qwen4_verifier.py:20-33 (_hyper) and patch_rmsnorm.py:108-135 (_rms_norm):
//
//   normed  = rms_norm(hidden)              mean of squares per group of gs
//                                           (gs = n: the whole row), fp32
//   d       = silu(W_down . normed / hc)    [lowrank], Q4/G32 vector form
//   mix     = sigmoid(W_up . d)             [n]
//   mixed   = mean_j(mix_j * normed_j)      [H], the branch input
//   weights = 2 * sigmoid(W_inj . normed / hc)   [hc]
//
// every step rounded to the activation type as MLX's bf16 arrays are.
//
//   k_hc_front  per token, blocks of four waves: the block normalises the
//               row into LDS (deterministic chunk sums of 64 squares, then one
//               wave sum per group), block 0 writes `normed`; each wave then
//               computes one row of W_down or W_inj against it.  The row's
//               weights, the streams and the gain are all loaded at entry.
//   k_hc_up     per token, a thread per output element h: the hc rows
//               j * H + h of W_up against d (staged in LDS), the sigmoid, the
//               products with the normalised streams and their mean; the
//               rows' first groups and the stream values load before d.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kHcThreads = 256;
constexpr int kHcWaves = kHcThreads / 64;

// Lanes without data load from here: every load is unconditional (a select
// of the address), so the loads issue back to back; a conditional load
// becomes a branch with a wait after it.
__device__ uint4 g_hc_zero[2];

__device__ __forceinline__ const void* or_zero(const void* p, bool live) {
  return live ? p : static_cast<const void*>(g_hc_zero);
}

// Eight consecutive activations (one 16-byte load in bf16, two in fp32),
// kept as raw bits until used.
template <class A>
struct Unit8 {
  uint4 a, b;
  __device__ __forceinline__ void load(const void* p, size_t i, bool live) {
    if constexpr (A::kBytes == 2) {
      a = ldg16(or_zero(static_cast<const uint16_t*>(p) + i, live));
    } else {
      a = ldg16(or_zero(static_cast<const float*>(p) + i, live));
      b = ldg16(or_zero(static_cast<const float*>(p) + i + 4, live));
    }
  }
  __device__ __forceinline__ float get(int k) const {
    if constexpr (A::kBytes == 2) {
      const uint32_t w = k < 2 ? a.x : k < 4 ? a.y : k < 6 ? a.z : a.w;
      return bf16_to_f32(k & 1 ? w >> 16 : w & 0xffffu);
    } else {
      const uint4& q = k < 4 ? a : b;
      const uint32_t w = (k & 3) == 0 ? q.x : (k & 3) == 1 ? q.y : (k & 3) == 2 ? q.z : q.w;
      return __uint_as_float(w);
    }
  }
};

template <class A>
__device__ __forceinline__ void store8(void* p, size_t i, const float y[8]) {
  if constexpr (A::kBytes == 2) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = f32_to_bf16(y[2 * k]) | (f32_to_bf16(y[2 * k + 1]) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    float4* q = reinterpret_cast<float4*>(static_cast<float*>(p) + i);
    q[0] = make_float4(y[0], y[1], y[2], y[3]);
    q[1] = make_float4(y[4], y[5], y[6], y[7]);
  }
}

// One Q4/G32 group in the vector form: s * sum(x * q) + b * sum(x).
__device__ __forceinline__ float q4_group(const uint4 words, float s, float b, const float* x) {
#pragma clang fp contract(off)
  const uint32_t w[4] = {words.x, words.y, words.z, words.w};
  float xq = 0.0f, xs = 0.0f;
#pragma unroll
  for (int k = 0; k < kGroup; ++k) {
    const float q = static_cast<float>((w[k / 8] >> (4 * (k % 8))) & 15u);
    xq = xq + x[k] * q;
    xs = xs + x[k];
  }
  return s * xq + b * xs;
}

constexpr int kHcUnits = kHcMaxRow / 8 / kHcThreads;     // 8-element units per thread
constexpr int kHcRowGroups = kHcMaxRow / kGroup / 64;    // Q4 groups of a projection row per lane

template <class A>
__global__ __launch_bounds__(kHcThreads) void k_hc_front(HcLaunch p) {
#pragma clang fp contract(off)
  // the normalised row, one pad float after every 32: lane l reads group
  // g = l + 64 i from s_x[33 g ...], a different bank for every lane
  __shared__ float s_x[kHcMaxRow + kHcMaxRow / kGroup];
  __shared__ float s_chunk[kHcMaxRow / 64];
  __shared__ float s_inv[kHcMaxRow / 64];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t t = blockIdx.y, n = p.n, gs = p.norm_group, r = p.lowrank, hc = p.hc;
  const size_t row_off = static_cast<size_t>(t) * n;
  const uint32_t units = n / 8, groups = n / kGroup;

  // 0. every load that does not depend on the norm, issued together: this
  //    wave's projection row (W_down rows 0..r-1, then W_inj rows), this
  //    thread's units of the streams and of the gain
  const uint32_t row = blockIdx.x * kHcWaves + wave;
  const bool live_row = row < r + hc;
  const bool down = row < r;
  const ProjPtrs pj = down ? p.down : p.inj;
  const uint32_t pr = down ? row : row - r;
  uint4 wq[kHcRowGroups];
  uint32_t wsb[kHcRowGroups], wbb[kHcRowGroups];
#pragma unroll
  for (int i = 0; i < kHcRowGroups; ++i) {
    const uint32_t g = lane + 64u * i;
    const bool live = live_row && g < groups;
    const size_t gi = static_cast<size_t>(pr) * groups + g;
    wq[i] = ldg16(or_zero(pj.w + gi * kWordsPerGroup, live));
    wsb[i] = ldg_u16(or_zero(pj.s + gi, live));
    wbb[i] = ldg_u16(or_zero(pj.b + gi, live));
  }
  Unit8<A> xu[kHcUnits], gu[kHcUnits];
#pragma unroll
  for (int i = 0; i < kHcUnits; ++i) {
    const uint32_t u = tid + kHcThreads * i;
    xu[i].load(p.hidden, row_off + 8 * u, u < units);
    gu[i].load(p.norm_weight, 8 * u, u < units);
  }

  // 1. sums of squares of every 64-element chunk (lanes 8c..8c+7 of a wave
  //    hold chunk c's eight units); n % 64 == 0 keeps those lanes together
#pragma unroll
  for (int i = 0; i < kHcUnits; ++i) {
    const uint32_t u = tid + kHcThreads * i;
    if (u >= units) break;  // uniform over each group of 8 lanes
    float sq = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) sq = sq + xu[i].get(k) * xu[i].get(k);
    sq = group_sum<8>(sq);
    if ((u & 7u) == 7u) s_chunk[u / 8] = sq;
  }
  lds_barrier();

  // 2. 1 / sqrt(mean + eps) of every group, one wave per group
  const uint32_t cpg = gs / 64;
  for (uint32_t g = wave; g < n / gs; g += kHcWaves) {
    float s = 0.0f;
    for (uint32_t c = lane; c < cpg; c += 64) s = s + s_chunk[g * cpg + c];
    s = wave_sum_all(s);
    if (lane == 0) s_inv[g] = 1.0f / sqrtf(s / static_cast<float>(gs) + p.eps);
  }
  lds_barrier();

  // 3. normalise: (x * inv) * gain, rounded to the activation type, into LDS
  //    (and block 0 of the token writes `normed`)
#pragma unroll
  for (int i = 0; i < kHcUnits; ++i) {
    const uint32_t u = tid + kHcThreads * i;
    if (u >= units) break;
    const float inv = s_inv[8 * u / gs];
    float y[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float w = gu[i].get(k);
      const float gain = p.one_centered ? w : 1.0f + w;
      y[k] = A::round((xu[i].get(k) * inv) * gain);
      s_x[8 * u + k + u / 4] = y[k];  // element e at e + e / 32
    }
    if (blockIdx.x == 0) store8<A>(p.normed, row_off + 8 * u, y);
  }
  lds_barrier();

  // 4. the wave's projection row against the normalised row
  if (!live_row) return;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kHcRowGroups; ++i) {
    const uint32_t g = lane + 64u * i;
    if (g < groups) acc = acc + q4_group(wq[i], bf16_to_f32(wsb[i]), bf16_to_f32(wbb[i]), s_x + g * (kGroup + 1));
  }
  acc = wave_sum_all(acc);
  if (lane != 0) return;
  const float a = A::round(A::round(acc) / static_cast<float>(hc));
  if (down) {
    A::store(p.d, static_cast<size_t>(t) * r + row, A::round(a * sigmoid_act<A>(a)));
  } else {
    A::store(p.weights, static_cast<size_t>(t) * hc + pr, A::round(2.0f * sigmoid_act<A>(a)));
  }
}

template <class A>
__global__ __launch_bounds__(kHcThreads) void k_hc_up(HcLaunch p) {
#pragma clang fp contract(off)
  __shared__ float s_d[kHcMaxLowrank];
  const uint32_t t = blockIdx.y, r = p.lowrank, hc = p.hc, H = p.width;
  const uint32_t h = blockIdx.x * kHcThreads + threadIdx.x;
  const bool live = h < H;
  const uint32_t groups = r / kGroup;
  // the first group of every stream's W_up row and the normalised stream
  // values, issued before the wait for d
  uint4 w0[kMaxStreams];
  uint32_t s0[kMaxStreams], b0[kMaxStreams], xn[kMaxStreams];
#pragma unroll
  for (int j = 0; j < static_cast<int>(kMaxStreams); ++j) {
    const bool lj = live && static_cast<uint32_t>(j) < hc;
    const size_t gi = (static_cast<size_t>(j) * H + h) * groups;
    w0[j] = ldg16(or_zero(p.up.w + gi * kWordsPerGroup, lj));
    s0[j] = ldg_u16(or_zero(p.up.s + gi, lj));
    b0[j] = ldg_u16(or_zero(p.up.b + gi, lj));
    const size_t xi = static_cast<size_t>(t) * p.n + j * H + h;
    xn[j] = A::kBytes == 2 ? ldg_u16(or_zero(static_cast<const uint16_t*>(p.normed) + xi, lj))
                           : ldg_u32(or_zero(static_cast<const float*>(p.normed) + xi, lj));
  }
  for (uint32_t k = threadIdx.x; k < r; k += kHcThreads) s_d[k] = A::load(p.d, static_cast<size_t>(t) * r + k);
  __syncthreads();
  if (!live) return;
  float total = 0.0f;
#pragma unroll
  for (int j = 0; j < static_cast<int>(kMaxStreams); ++j) {
    if (static_cast<uint32_t>(j) >= hc) break;
    const size_t gi = (static_cast<size_t>(j) * H + h) * groups;
    float acc = q4_group(w0[j], bf16_to_f32(s0[j]), bf16_to_f32(b0[j]), s_d);
    for (uint32_t g = 1; g < groups; ++g)
      acc = acc + q4_group(ldg16(p.up.w + (gi + g) * kWordsPerGroup), bf16_to_f32(ldg_u16(p.up.s + gi + g)),
                           bf16_to_f32(ldg_u16(p.up.b + gi + g)), s_d + g * kGroup);
    const float mix = sigmoid_act<A>(A::round(acc));
    total = total + A::round(mix * A::from_bits(xn[j]));
  }
  A::store(p.mixed, static_cast<size_t>(t) * H + h, A::round(A::round(total) * A::round(1.0f / static_cast<float>(hc))));
}

template <class K>
hipError_t launch_timed(const char* family, K kernel, dim3 grid, const HcLaunch& p, hipStream_t stream) {
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events(family, &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, dim3(kHcThreads), 0, stream, start, stop, 0, p);
  else
    hipLaunchKernelGGL(kernel, grid, dim3(kHcThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_hyper_mix(const HcLaunch& p, hipStream_t stream) {
  const dim3 front((p.lowrank + p.hc + kHcWaves - 1) / kHcWaves, p.tokens);
  const dim3 up((p.width + kHcThreads - 1) / kHcThreads, p.tokens);
  hipError_t e = p.act_dtype == 0 ? launch_timed("hc_front", k_hc_front<ActBF16>, front, p, stream)
                                  : launch_timed("hc_front", k_hc_front<ActF32>, front, p, stream);
  if (e != hipSuccess) return e;
  return p.act_dtype == 0 ? launch_timed("hc_up", k_hc_up<ActBF16>, up, p, stream)
                          : launch_timed("hc_up", k_hc_up<ActF32>, up, p, stream);
}

}  // namespace vm

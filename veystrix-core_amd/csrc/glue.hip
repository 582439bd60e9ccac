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
//               computes one row of W_down or W_inj against it.
//   k_hc_up     per token, a thread per output element h: the hc rows
//               j * H + h of W_up against d (staged in LDS), the sigmoid, the
//               products with the normalised streams and their mean.
#include <hip/hip_runtime.h>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kHcThreads = 256;
constexpr int kHcWaves = kHcThreads / 64;

template <class A>
__device__ __forceinline__ void load8(const void* p, size_t i, float v[8]) {
  if constexpr (A::kBytes == 2) {
    const uint4 q = ldg16(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = bf16_to_f32(k & 1 ? w[k / 2] >> 16 : w[k / 2] & 0xffffu);
  } else {
    const uint4 a = ldg16(static_cast<const float*>(p) + i);
    const uint4 b = ldg16(static_cast<const float*>(p) + i + 4);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = __uint_as_float(w[k]);
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

template <class A>
__global__ __launch_bounds__(kHcThreads) void k_hc_front(HcLaunch p) {
#pragma clang fp contract(off)
  __shared__ float s_x[kHcMaxRow];
  __shared__ float s_chunk[kHcMaxRow / 64];
  __shared__ float s_inv[kHcMaxRow / 64];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t t = blockIdx.y, n = p.n, gs = p.norm_group, r = p.lowrank, hc = p.hc;
  const size_t row_off = static_cast<size_t>(t) * n;

  // 1. the row into LDS; sums of squares of every 64-element chunk (lanes
  //    8c..8c+7 of a wave hold chunk c's eight 8-element units)
  for (uint32_t u = tid; u < n / 8; u += kHcThreads) {
    float v[8];
    load8<A>(p.hidden, row_off + 8 * u, v);
    float sq = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      s_x[8 * u + k] = v[k];
      sq = sq + v[k] * v[k];
    }
    sq = group_sum<8>(sq);
    if ((u & 7u) == 7u) s_chunk[u / 8] = sq;
  }
  __syncthreads();

  // 2. 1 / sqrt(mean + eps) of every group, one wave per group
  const uint32_t cpg = gs / 64;
  for (uint32_t g = wave; g < n / gs; g += kHcWaves) {
    float s = 0.0f;
    for (uint32_t c = lane; c < cpg; c += 64) s = s + s_chunk[g * cpg + c];
    s = wave_sum_all(s);
    if (lane == 0) s_inv[g] = 1.0f / sqrtf(s / static_cast<float>(gs) + p.eps);
  }
  __syncthreads();

  // 3. normalise in place: (x * inv) * gain, rounded to the activation type
  for (uint32_t i = tid; i < n; i += kHcThreads) {
    const float w = A::load(p.norm_weight, i);
    const float gain = p.one_centered ? w : 1.0f + w;
    const float y = A::round((s_x[i] * s_inv[i / gs]) * gain);
    s_x[i] = y;
    if (blockIdx.x == 0) A::store(p.normed, row_off + i, y);
  }
  __syncthreads();

  // 4. one projection row per wave: W_down rows 0..r-1, then W_inj rows
  const uint32_t row = blockIdx.x * kHcWaves + wave;
  if (row >= r + hc) return;
  const bool down = row < r;
  const ProjPtrs& pj = down ? p.down : p.inj;
  const uint32_t pr = down ? row : row - r;
  const uint32_t groups = n / kGroup;
  float acc = 0.0f;
  for (uint32_t g = lane; g < groups; g += 64) {
    const size_t gi = static_cast<size_t>(pr) * groups + g;
    const uint4 words = ldg16(pj.w + gi * kWordsPerGroup);
    acc = acc + q4_group(words, bf16_to_f32(ldg_u16(pj.s + gi)), bf16_to_f32(ldg_u16(pj.b + gi)), s_x + g * kGroup);
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
  for (uint32_t k = threadIdx.x; k < r; k += kHcThreads) s_d[k] = A::load(p.d, static_cast<size_t>(t) * r + k);
  __syncthreads();
  const uint32_t h = blockIdx.x * kHcThreads + threadIdx.x;
  if (h >= H) return;
  const uint32_t groups = r / kGroup;
  float total = 0.0f;
  for (uint32_t j = 0; j < hc; ++j) {
    const uint32_t o = j * H + h;
    float acc = 0.0f;
    for (uint32_t g = 0; g < groups; ++g) {
      const size_t gi = static_cast<size_t>(o) * groups + g;
      const uint4 words = ldg16(p.up.w + gi * kWordsPerGroup);
      acc = acc + q4_group(words, bf16_to_f32(ldg_u16(p.up.s + gi)), bf16_to_f32(ldg_u16(p.up.b + gi)), s_d + g * kGroup);
    }
    const float mix = sigmoid_act<A>(A::round(acc));
    total = total + A::round(mix * A::load(p.normed, static_cast<size_t>(t) * p.n + o));
  }
  A::store(p.mixed, static_cast<size_t>(t) * H + h, A::round(A::round(total) * A::round(1.0f / static_cast<float>(hc))));
}

template <class K>
hipError_t launch_plain(K kernel, dim3 grid, const HcLaunch& p, hipStream_t stream) {
  hipLaunchKernelGGL(kernel, grid, dim3(kHcThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_hyper_mix(const HcLaunch& p, hipStream_t stream) {
  const dim3 front((p.lowrank + p.hc + kHcWaves - 1) / kHcWaves, p.tokens);
  const dim3 up((p.width + kHcThreads - 1) / kHcThreads, p.tokens);
  hipError_t e = p.act_dtype == 0 ? launch_plain(k_hc_front<ActBF16>, front, p, stream)
                                  : launch_plain(k_hc_front<ActF32>, front, p, stream);
  if (e != hipSuccess) return e;
  return p.act_dtype == 0 ? launch_plain(k_hc_up<ActBF16>, up, p, stream)
                          : launch_plain(k_hc_up<ActF32>, up, p, stream);
}

}  // namespace vm

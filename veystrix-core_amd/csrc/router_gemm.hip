// Router logits of grouped calls (more than 64 rows) for gfx950: fp32
// [T, E] = round_bf16(x . W^T + bias), x bf16 [T, K], W bf16 [E, K].
//
// A plain bf16 GEMM with a short K loop per output tile: with the weights'
// loads one chunk ahead (the Q4 GEMMs' scheme) every chunk waited out a full
// load latency.  Here both operands stream global -> LDS directly
// (global_load_lds_dwordx4: no registers held, no copy through VGPRs) into a
// ring of S stages of 64 K-inputs each, so S - 1 stages are in flight while
// one is multiplied.
//
//   tile     64 TM rows x 64 TM columns per 4-wave block (TM = 1 or 2);
//            wave (wm, wn) owns rows 32 TM wm .. +32 TM and as many columns
//            from 32 TM wn (2 TM by 2 TM MFMA blocks of 16 x 16), so a K step
//            reads 2 TM A and 2 TM B fragments for 4 TM^2
//            v_mfma_f32_16x16x32_bf16.  TM = 2 halves the rows and router
//            rows that reach LDS per logit (each is read once per tile of the
//            other operand); it is used while it still gives every CU a block.
//   stage    A rows then W rows, 128 bytes (64 inputs) each: TM (8 KB + 8 KB).
//            The 16-byte unit u of row r sits at unit u ^ swz(r), swz(r)
//            moving row bits 2 and 1 onto unit bits 1 and 2.  An MFMA read
//            (lane l: row l % 16, unit 4 ks + l / 16) then lands on the bank
//            slot (r0, akb0, akb1 ^ r2, r1) of the 512-byte-row layout of the
//            Q4 GEMMs, which is conflict-free for every lane grouping that
//            layout was measured against.  A DMA instruction writes 1 KB of
//            consecutive LDS (lane j -> bytes 16 j), eight rows: its lanes
//            load their row's units in the swizzled order, so the XOR is paid
//            once per load, on the global side.
//   ring     one __shared__ array per stage: the compiler tracks each
//            stage's DMA writes separately and waits only for the stage a
//            read needs (one array for the ring made it wait for every load
//            in flight before each read).  The barrier is a bare s_barrier:
//            __syncthreads()'s release fence would wait for the DMA loads
//            in flight as well.
//   order    blocks are dealt to the eight XCDs round-robin; the column
//            slices of one row tile take blocks of one XCD, which then reads
//            the tile's rows from HBM once and from its L2 after that.
//
// Each logit sums its K inputs in the same order at every row count (the
// same lanes, steps and stages for every tile), so a token's experts do not
// depend on how many rows its call has.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "vm_internal.h"

namespace vm {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kRtK = 64;           // K inputs per stage
constexpr int kRtRowBytes = kRtK * 2;
constexpr int kRtThreads = 256;
// Tile of TM x 64 rows by TM x 64 columns (TM = 1 or 2); a stage holds its A
// rows then its router rows, 128 bytes each: TM x 16 KB.
template <int TM>
constexpr int rt_tile() {
  return 64 * TM;
}
template <int TM>
constexpr int rt_half() {
  return rt_tile<TM>() * kRtRowBytes;
}
template <int TM>
constexpr int rt_dma_per_wave() {  // 1 KB DMA loads per wave and stage
  return 2 * rt_half<TM>() / 1024 / (kRtThreads / 64);
}
static_assert(rt_dma_per_wave<1>() == 4 && rt_dma_per_wave<2>() == 8, "whole 1 KB loads per wave");

__device__ __forceinline__ uint32_t rt_swz(uint32_t r) { return ((r >> 1) & 2u) | ((r << 1) & 4u); }

// Stage J of the ring: one LDS object per stage.
template <int J, int TM>
__device__ __forceinline__ uint8_t* rt_stage() {
  __shared__ uint4 buf[2 * rt_half<TM>() / 16];
  return reinterpret_cast<uint8_t*>(buf);
}

template <int J, int N, class F>
__device__ __forceinline__ void rt_unroll(F&& f) {
  if constexpr (J < N) {
    f(std::integral_constant<int, J>{});
    rt_unroll<J + 1, N>(f);
  }
}

// s_waitcnt for vmcnt(N) only (expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4)); }

// The barrier between stages.  The empty asm statements keep the compiler
// from moving LDS accesses across it (s_barrier itself is not a memory
// operation to the compiler).
__device__ __forceinline__ void rt_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int S, int NST, int TM>
__global__ __launch_bounds__(kRtThreads) void k_router_gemm(GroupedLaunch p) {
  constexpr int kTile = rt_tile<TM>(), kHalf = rt_half<TM>(), kDma = rt_dma_per_wave<TM>();
  constexpr int kB = 2 * TM;  // 16-row (and 16-column) MFMA blocks per wave
  constexpr uint32_t kAGroups = kTile / 8;  // 1 KB loads of the A rows per stage
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t T = p.rows, K = p.k_dim, E = p.n_dim;
  const uint32_t slices = E / kTile;
  const uint32_t row_tiles = (T + kTile - 1) / kTile;
  const uint32_t lin = blockIdx.x, local = lin >> 3;
  const uint32_t tile = (local / slices) * 8u + (lin & 7u), slice = local % slices;
  if (blockIdx.x == 0 && p.zero_words != nullptr) {
    for (uint32_t i = tid; i < p.zero_count; i += kRtThreads) p.zero_words[i] = 0;
    wait_vm<0>();  // the stores leave the vector memory count before the DMA loads are counted
  }
  if (tile >= row_tiles) return;
  const uint32_t row0 = tile * kTile, col0 = slice * kTile;

  // DMA loads: load i of this wave is 1 KB number g = kDma wave + i of the
  // stage (A rows 8 g .. +8 for g < kAGroups, else router rows 8 (g -
  // kAGroups) .. +8); lane j loads unit (j % 8) ^ swz(row) of that row
  // group's row j / 8 into bytes 16 j.
  uint32_t g_off[kDma];  // byte offsets from the matrix at K input 0
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    const uint32_t g = wave * kDma + i;
    const uint32_t r = 8u * (g % kAGroups) + lane / 8u;
    const uint32_t u = (lane % 8u) ^ rt_swz(r);
    const uint32_t src = g < kAGroups ? min(row0 + r, T - 1u) : col0 + r;
    g_off[i] = (src * K + u * 8u) * 2u;
  }
  const uint8_t* xa = reinterpret_cast<const uint8_t*>(p.a);
  const uint8_t* wb = reinterpret_cast<const uint8_t*>(p.bf16_weight);
  static_assert(NST >= S && S >= 2, "the ring is filled before the first stage");
  static_assert((S - 2) * kDma < 64, "the ring's loads fit the vector memory count");
  auto issue = [&](auto J, uint32_t c) {
    uint8_t* st = rt_stage<decltype(J)::value, TM>();
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      const uint32_t g = wave * kDma + i;  // wave-uniform
      const uint8_t* src = (g < kAGroups ? xa : wb) + c * kRtRowBytes + g_off[i];
      __builtin_amdgcn_global_load_lds(
          src, (__attribute__((address_space(3))) void*)(st + (g % kAGroups) * 1024u + (g < kAGroups ? 0u : kHalf)),
          16, 0, 0);
    }
  };

  // MFMA reads: lane -> (row or column lane % 16, K block lane / 16)
  const uint32_t wm = wave & 1u, wn = wave >> 1;
  const uint32_t lm = lane & 15u, kb = lane >> 4;
  const uint32_t s = rt_swz(lm);  // rows 16 b + lm have the swizzle of lm
  const uint32_t u0 = (kb ^ s) * 16u, u1 = ((4u | kb) ^ s) * 16u;
  const uint32_t a_base = (16u * kB * wm + lm) * kRtRowBytes;
  const uint32_t b_base = kHalf + (16u * kB * wn + lm) * kRtRowBytes;
  // the bias of the lane's output columns, loaded before the K loop
  float bias[kB];
#pragma unroll
  for (int j = 0; j < kB; ++j) bias[j] = p.bias != nullptr ? p.bias[col0 + 16u * kB * wn + 16u * j + lm] : 0.0f;
  f32x4_t acc[kB][kB];
#pragma unroll
  for (int i = 0; i < kB; ++i)
#pragma unroll
    for (int j = 0; j < kB; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](auto J) {
    const uint8_t* st = rt_stage<decltype(J)::value, TM>();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const uint32_t u = ks ? u1 : u0;
      bf16x8_t a[kB], b[kB];
#pragma unroll
      for (int i = 0; i < kB; ++i) {
        a[i] = *reinterpret_cast<const bf16x8_t*>(st + a_base + i * 16 * kRtRowBytes + u);
        b[i] = *reinterpret_cast<const bf16x8_t*>(st + b_base + i * 16 * kRtRowBytes + u);
      }
#pragma unroll
      for (int i = 0; i < kB; ++i)
#pragma unroll
        for (int j = 0; j < kB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };

  // prologue: stages 0 .. S-2 in flight.  The K loop is unrolled whole (NST
  // stages, a compile-time count): at the head of a rolled loop the compiler
  // could not tell which stage's loads a read needs and waited for all of
  // them once per turn of the ring.
  rt_unroll<0, S - 1>([&](auto J) { issue(J, decltype(J)::value); });
  rt_unroll<0, NST>([&](auto C) {
    constexpr int c = decltype(C)::value;
    // this wave's loads of stage c are done once only the later stages' remain
    wait_vm<(c + S - 2 < NST ? S - 2 : NST - 1 - c) * kDma>();
    wait_lgkm0();  // this wave's reads of stage c - 1 are done before its slot is refilled
    rt_barrier();  // every wave's loads of stage c have landed
    if constexpr (c + S - 1 < NST) issue(std::integral_constant<int, (c + S - 1) % S>{}, c + S - 1);
    compute(std::integral_constant<int, c % S>{});
  });

  // lane holds C[4 (lane / 16) + q][lane % 16] of each 16 x 16 block
#pragma unroll
  for (int j = 0; j < kB; ++j) {
    const uint32_t col = col0 + 16u * kB * wn + 16u * j + lm;
#pragma unroll
    for (int i = 0; i < kB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t row = row0 + 16u * kB * wm + 16u * i + 4u * kb + q;
        if (row < T) static_cast<float*>(p.out)[row * E + col] = round_bf16(acc[i][j][q] + bias[j]);
      }
  }
}

template <class... KArgs, class... Args>
hipError_t rt_launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, Args... args) {
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events("router_gemm", &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
  return hipGetLastError();
}

}  // namespace

bool router_gemm_supported(uint32_t k_dim, uint32_t n_dim) {
  return (k_dim == 1024 || k_dim == 2048 || k_dim == 4096) && n_dim % rt_tile<1>() == 0 && n_dim > 0;
}

#ifndef VM_ROUTER_BIG_TILE
#define VM_ROUTER_BIG_TILE 1
#endif
// Ring depths: 64 x 64 tiles at one block per CU, and 128 x 128 tiles.
#ifndef VM_ROUTER_STAGES_1
#define VM_ROUTER_STAGES_1 8
#endif
#ifndef VM_ROUTER_STAGES_2
#define VM_ROUTER_STAGES_2 4
#endif

template <int NST>
hipError_t router_gemm_go(const GroupedLaunch& p, hipStream_t stream) {
  auto blocks = [&](uint32_t tile) {
    const uint32_t row_tiles = (p.rows + tile - 1) / tile, slices = p.n_dim / tile;
    return std::make_pair(row_tiles * slices, (row_tiles + 7u) / 8u * 8u * slices);
  };
  // 128 x 128 tiles with four stages (one block per CU) once they still give
  // every CU a block: half the L2 -> LDS traffic of 64 x 64 tiles, which
  // re-read the rows once per 64 columns and the router rows once per 64 rows
  const auto big = blocks(rt_tile<2>());
  if (VM_ROUTER_BIG_TILE && p.n_dim % rt_tile<2>() == 0 && big.first >= 256u)
    return rt_launch(k_router_gemm<VM_ROUTER_STAGES_2, NST, 2>, dim3(big.second), dim3(kRtThreads), stream, p);
  // 64 x 64 tiles: eight stages and one block per CU while the grid is at
  // most one block per CU; above that four stages, two blocks per CU
  const auto small = blocks(rt_tile<1>());
  if (small.first <= 256u)
    return rt_launch(k_router_gemm<VM_ROUTER_STAGES_1, NST, 1>, dim3(small.second), dim3(kRtThreads), stream, p);
  return rt_launch(k_router_gemm<4, NST, 1>, dim3(small.second), dim3(kRtThreads), stream, p);
}

hipError_t launch_router_gemm(const GroupedLaunch& p, hipStream_t stream) {
  if (!router_gemm_supported(p.k_dim, p.n_dim) || p.rows == 0 ||
      static_cast<uint64_t>(p.rows) * p.k_dim * 2u > 0xffffffffull ||
      static_cast<uint64_t>(p.rows) * p.n_dim > 0xffffffffull || p.a_stride != p.k_dim)
    return hipErrorInvalidValue;
  switch (p.k_dim) {
    case 1024: return router_gemm_go<1024 / kRtK>(p, stream);
    case 2048: return router_gemm_go<2048 / kRtK>(p, stream);
    default: return router_gemm_go<4096 / kRtK>(p, stream);
  }
}

}  // namespace vm

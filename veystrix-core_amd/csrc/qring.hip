// Q4/G32 grouped GEMM of calls above 64 rows (the gate/up + SwiGLU and the
// down projections of chunked prefill) with every operand streamed global ->
// LDS by the DMA path (global_load_lds): the gathered activation rows, the
// packed weight lines and the scale and bias vectors land in a ring of S
// stages without passing through registers, so a block holds no prefetch
// registers, issues no LDS stores and keeps S - 1 stages in flight.
//
//   tile     up to 64 rows of one expert group (MBU 16-row MFMA blocks) by
//            128 weight rows: 64 gate + 64 up features (four waves, each
//            16 + 16) or 128 down features (each wave 32).  Every wave takes
//            all rows of its columns, so a column's weights are dequantised
//            once per tile.
//   stage    128 inputs (four 32-input groups): A rows 256 bytes each, weight
//            lines 64 bytes each, scales and biases 8 bytes each per weight
//            row: 26 KB at 64 rows.
//   dequant  per 8 inputs of a lane: four v_and_or into f16 magic pairs,
//            eight v_fma_mix (w = s q + b exactly as s (1024 + q) + (b - 1024
//            s), or (s / 16) (1024 + 16 q) + (b - 64 s) for the high nibble
//            of a byte), four v_cvt_pk_bf16_f32 pairing the results in input
//            order, so the A rows are used as stored.
//   banks    a ds_read_b128 of 64 lanes is served a few lanes groups at a
//            time; the 16-byte units of a row are XOR-swizzled with row bits
//            so that lanes 0-3 of a group (row bits 0, 1) and its k blocks or
//            row bits 2, 3 fall on distinct bank groups (A: unit u of tile
//            row r at u ^ a_swz(r); weights: group g of weight row c at
//            g ^ w_swz(c)).  A DMA instruction writes 1 KB of consecutive
//            LDS, so the lanes load the swizzled units' global addresses.
//   ring     one __shared__ array per stage, so the compiler's waits follow
//            each stage's DMA writes; a bare s_barrier between stages (the
//            fence of __syncthreads() would wait for every DMA in flight);
//            the K loop unrolled whole.
//   order    the XCD-aware tile order of the chunked GEMM: XCD x takes the
//            x-th eighth of the sorted tiles, each with all its column slices.
//
// The fp32 sums follow a fixed lane and step order at every row count, so a
// row's outputs do not depend on the call it is in.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <type_traits>
#include <utility>

#include "vm_internal.h"

namespace vm {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kQrWaves = 4;
constexpr int kQrThreads = kQrWaves * 64;
constexpr int kQrGroups = 4;                  // 32-input groups per stage
constexpr int kQrK = kQrGroups * kGroup;      // 128 inputs per stage
constexpr int kQrRowBytes = kQrK * 2;         // A bytes per row and stage
constexpr int kQrTileRows = 64;               // rows per tile at most
constexpr int kQrWRows = 128;                 // weight rows per block
constexpr int kQrWLine = kQrK / 2;            // 64 bytes of packed weights per row and stage
constexpr int kQrABytes = kQrTileRows * kQrRowBytes;   // 16 KB
constexpr int kQrWBytes = kQrWRows * kQrWLine;         // 8 KB
constexpr int kQrSBytes = kQrWRows * kQrGroups * 2;    // 1 KB of scales (and of biases)
constexpr int kQrWSlot = kQrWBytes + 2 * kQrSBytes;     // weights, scales, biases of a stage
static_assert(kQrWSlot == 10 * 1024, "a weight slot is 10 KB");
static_assert(kQrWBytes / 1024 == 2 * kQrWaves && kQrSBytes / 256 == kQrWaves, "whole DMA units per wave");

// Ring depths: activation rows (16 KB slots, read from the L2) and weights
// (10 KB slots, read from HBM).  2 and 4: 72 KB of LDS, two blocks per CU,
// three stages of weights in flight per block.
#ifndef VM_QR_ASLOTS
#define VM_QR_ASLOTS 2
#endif
#ifndef VM_QR_WSLOTS
#define VM_QR_WSLOTS 4
#endif
#ifndef VM_QRING_DEFAULT
#define VM_QRING_DEFAULT 0
#endif

__device__ __forceinline__ constexpr uint32_t qr_a_swz(uint32_t r) {
  return (r & 3u) | ((r >> 1) & 4u) | ((r << 1) & 8u);
}
__device__ __forceinline__ constexpr uint32_t qr_w_swz(uint32_t c) { return ((c >> 3) & 1u) | ((c >> 1) & 2u); }

// Slot J of the activation ring and of the weight ring: one LDS object per
// slot, so the compiler's waits follow each slot's DMA writes.
template <int J>
__device__ __forceinline__ uint8_t* qr_aslot() {
  __shared__ uint4 buf[kQrABytes / 16];
  return reinterpret_cast<uint8_t*>(buf);
}
template <int J>
__device__ __forceinline__ uint8_t* qr_wslot() {
  __shared__ uint4 buf[kQrWSlot / 16];
  return reinterpret_cast<uint8_t*>(buf);
}

// The vector-memory count to wait for at the head of stage c, so that this
// wave's DMA loads of stage c (its activation rows and its weights) have
// landed: loads complete in issue order, so it is the number of loads this
// wave issued after the last of them.  Issue order: the prologue takes i = 0
// .. SW - 2 as [A(i) if i < SA - 1] [W(i)]; the head of stage k then issues
// A(k + SA - 1) and W(k + SW - 1) (those below NST), nA and nW loads each.
constexpr int qr_wait_for(int c, int SA, int SW, int NST, int nA, int nW) {
  int after = 0;
  for (int k = c - 1; k >= 0; --k) {
    if (k + SW - 1 < NST) {
      if (k + SW - 1 == c) return after;
      after += nW;
    }
    if (k + SA - 1 < NST) {
      if (k + SA - 1 == c) return after;
      after += nA;
    }
  }
  for (int i = SW - 2; i >= 0; --i) {
    if (i < NST) {
      if (i == c) return after;
      after += nW;
    }
    if (i < SA - 1 && i < NST) {
      if (i == c) return after;
      after += nA;
    }
  }
  return 0;
}

template <int J, int N, class F>
__device__ __forceinline__ void qr_unroll(F&& f) {
  if constexpr (J < N) {
    f(std::integral_constant<int, J>{});
    qr_unroll<J + 1, N>(f);
  }
}

template <int N>
__device__ __forceinline__ void qr_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void qr_wait_lgkm0() { __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4)); }

__device__ __forceinline__ void qr_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t qr_pack(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t qr_magic() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}

__device__ __forceinline__ uint32_t qr_opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// A wave-uniform address held in SGPRs from here on.
__device__ __forceinline__ const uint8_t* qr_sbase(const uint8_t* p) {
  asm volatile("" : "+s"(p));
  return p;
}

// The affine constants of one group: w = s q + b for q = the low nibble of
// a byte as s (1024 + q) + (b - 1024 s), for the high one as (s / 16)
// (1024 + 16 q) + (b - 64 s); (1024 + q) and (1024 + 16 q) are exact f16.
struct QrAffine {
  float s, b1024, s16, b64;
  __device__ __forceinline__ void set(float scale, float bias) {
    s = scale;
    b1024 = fmaf(-1024.0f, scale, bias);
    s16 = 0.0625f * scale;
    b64 = fmaf(-64.0f, scale, bias);
  }
  // the 8 inputs of one packed word as bf16 in input order
  __device__ __forceinline__ bf16x8_t word(uint32_t w, uint32_t magic) const {
    const uint32_t w8 = w >> 8;
    const f16x2_t m0 = __builtin_bit_cast(f16x2_t, (w & 0x000F000Fu) | magic);   // q0, q4
    const f16x2_t m1 = __builtin_bit_cast(f16x2_t, (w & 0x00F000F0u) | magic);   // 16 q1, 16 q5
    const f16x2_t m2 = __builtin_bit_cast(f16x2_t, (w8 & 0x000F000Fu) | magic);  // q2, q6
    const f16x2_t m3 = __builtin_bit_cast(f16x2_t, (w8 & 0x00F000F0u) | magic);  // 16 q3, 16 q7
    const float v0 = fmaf(s, static_cast<float>(m0.x), b1024), v4 = fmaf(s, static_cast<float>(m0.y), b1024);
    const float v1 = fmaf(s16, static_cast<float>(m1.x), b64), v5 = fmaf(s16, static_cast<float>(m1.y), b64);
    const float v2 = fmaf(s, static_cast<float>(m2.x), b1024), v6 = fmaf(s, static_cast<float>(m2.y), b1024);
    const float v3 = fmaf(s16, static_cast<float>(m3.x), b64), v7 = fmaf(s16, static_cast<float>(m3.y), b64);
    const uint4 r = make_uint4(qr_pack(v0, v1), qr_pack(v2, v3), qr_pack(v4, v5), qr_pack(v6, v7));
    return __builtin_bit_cast(bf16x8_t, r);
  }
};

__device__ __forceinline__ void qr_flag(uint32_t* status, uint32_t bits) {
  if (status != nullptr) atomicOr(status, bits);
}

// One tile (rows [row0, row0 + rows) of one group, MBU = ceil(rows / 16))
// by the 128 weight rows of column slice `slice`: NST stages of 128 inputs.
// PROJ 2: gate and up (64 features each, SwiGLU epilogue); PROJ 1: 128
// features of one projection (bf16 rows).
template <int EPI, int MBU, int SA, int SW, int NST>
__device__ __forceinline__ void qr_tile(const GroupedLaunch& p, const ProjPtrs* w, uint32_t row0, uint32_t rows,
                                        uint32_t slice) {
  constexpr int PROJ = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int kCols = kQrWRows / PROJ;     // features per projection and block
  constexpr int NBW = kCols / (kQrWaves * 16);  // 16-column MFMA blocks per wave and projection
  constexpr int nA = MBU, nW = 4;            // DMA instructions per wave and stage: activations, weights
  static_assert(SA >= 2 && SW >= SA && NST >= SW - 1, "the rings are filled before the first stage");
  static_assert((SA - 1) * nA + (SW - 1) * nW < 64, "the rings' loads fit the vector memory count");
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t K = p.k_dim, N = p.n_dim, G = K / kGroup;

  // ---- DMA sources: wave w issues units w, w + 4, ... of the stage: MBU A
  // units (4 rows each), 2 weight units (16 weight rows each), one scale and
  // one bias unit (32 weight rows of 8 bytes each, dword DMA).
  uint32_t a_off[MBU];
#pragma unroll
  for (int j = 0; j < MBU; ++j) {
    const uint32_t r = 16u * j + 4u * wave + lane / 16u;  // tile row (unit 4 j + wave holds rows 16 j + 4 wave ..)
    const uint32_t rr = r < rows ? r : 0u;
    const uint32_t arow = p.row_token != nullptr ? p.row_token[row0 + rr] : row0 + rr;
    const uint32_t u = (lane & 15u) ^ qr_a_swz(r & 15u);
    a_off[j] = (arow * p.a_stride + u * 8u) * 2u;
  }
  // weight row rho = 16 (4 i + wave) + lane / 4 of the block, i < 2
  const uint8_t* w_base[2];
  uint32_t w_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t rho = 16u * (4u * i + wave) + lane / 4u;
    const int pj = PROJ == 2 ? i : 0;
    const uint32_t col = min(slice * kCols + rho % kCols, N - 1u);
    const uint32_t g = (lane & 3u) ^ qr_w_swz(rho & 15u);
    w_base[i] = reinterpret_cast<const uint8_t*>(w[pj].w);
    w_off[i] = col * (K / 2u) + g * 16u;
  }
  // scale and bias rows rho = 32 wave + lane / 2, dword lane & 1
  const uint32_t s_rho = 32u * wave + lane / 2u;
  const uint32_t s_pj = PROJ == 2 ? (32u * wave) / kCols : 0u;  // wave-uniform
  const uint8_t* s_base = reinterpret_cast<const uint8_t*>(s_pj ? w[PROJ - 1].s : w[0].s);
  const uint8_t* b_base = reinterpret_cast<const uint8_t*>(s_pj ? w[PROJ - 1].b : w[0].b);
  const uint32_t s_off = min(slice * kCols + s_rho % kCols, N - 1u) * G * 2u + (lane & 1u) * 4u;
  const uint8_t* a_base = reinterpret_cast<const uint8_t*>(p.a);

  // a stage's source of each unit: a base in SGPRs, moved on by the stage
  // (scalar adds), plus the lane's 32-bit offset (the saddr form, no 64-bit
  // address arithmetic per load)
  auto issue_a = [&](auto J, uint32_t c) {
    uint8_t* st = qr_aslot<decltype(J)::value>();
    const uint8_t* ab = qr_sbase(a_base + c * kQrRowBytes);
#pragma unroll
    for (int j = 0; j < MBU; ++j)
      __builtin_amdgcn_global_load_lds(ab + qr_opaque(a_off[j]),
                                       (__attribute__((address_space(3))) void*)(st + (4u * j + wave) * 1024u), 16,
                                       0, 0);
  };
  auto issue_w = [&](auto J, uint32_t c) {
    uint8_t* st = qr_wslot<decltype(J)::value>();
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(qr_sbase(w_base[i] + c * kQrWLine) + qr_opaque(w_off[i]),
                                       (__attribute__((address_space(3))) void*)(st + (4u * i + wave) * 1024u), 16,
                                       0, 0);
    __builtin_amdgcn_global_load_lds(qr_sbase(s_base + c * (kQrGroups * 2)) + qr_opaque(s_off),
                                     (__attribute__((address_space(3))) void*)(st + kQrWBytes + wave * 256u), 4, 0,
                                     0);
    __builtin_amdgcn_global_load_lds(qr_sbase(b_base + c * (kQrGroups * 2)) + qr_opaque(s_off),
                                     (__attribute__((address_space(3))) void*)(st + kQrWBytes + kQrSBytes +
                                                                               wave * 256u),
                                     4, 0, 0);
  };

  // ---- MFMA reads: lane -> (row or column lane % 16, k block lane / 16)
  const uint32_t lm = lane & 15u, kb = lane >> 4;
  // A: tile row 16 mb + lm, logical unit 4 kb + st of the stage
  uint32_t a_rd[4];
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) a_rd[s4] = lm * kQrRowBytes + (((4u * kb + s4) ^ qr_a_swz(lm)) * 16u);
  // weights: block row rho(pj, nb) = pj kCols + wave NBW 16 + nb 16 + lm, group kb
  const uint32_t w_rd = (wave * NBW * 16u + lm) * kQrWLine + ((kb ^ qr_w_swz(lm)) * 16u);
  const uint32_t s_rd = kQrWBytes + (wave * NBW * 16u + lm) * (kQrGroups * 2) + kb * 2u;

  f32x4_t acc[PROJ][NBW][MBU];
#pragma unroll
  for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
      for (int mb = 0; mb < MBU; ++mb) acc[pj][nb][mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t magic = qr_magic();

  auto compute = [&](auto JA, auto JW) {
    const uint8_t* sa = qr_aslot<decltype(JA)::value>();
    const uint8_t* st = qr_wslot<decltype(JW)::value>();
    uint4 wv[PROJ][NBW];
    QrAffine af[PROJ][NBW];
#pragma unroll
    for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        const uint32_t ro = (pj * kCols + nb * 16u);
        wv[pj][nb] = *reinterpret_cast<const uint4*>(st + w_rd + ro * kQrWLine);
        const uint32_t sb = *reinterpret_cast<const uint16_t*>(st + s_rd + ro * (kQrGroups * 2));
        const uint32_t bb = *reinterpret_cast<const uint16_t*>(st + s_rd + kQrSBytes + ro * (kQrGroups * 2));
        af[pj][nb].set(__uint_as_float(sb << 16), __uint_as_float(bb << 16));
      }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      bf16x8_t a[MBU];
#pragma unroll
      for (int mb = 0; mb < MBU; ++mb)
        a[mb] = *reinterpret_cast<const bf16x8_t*>(sa + a_rd[s4] + mb * 16 * kQrRowBytes);
#pragma unroll
      for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
          const uint32_t word = s4 == 0 ? wv[pj][nb].x : s4 == 1 ? wv[pj][nb].y : s4 == 2 ? wv[pj][nb].z : wv[pj][nb].w;
          const bf16x8_t b = af[pj][nb].word(word, magic);
#pragma unroll
          for (int mb = 0; mb < MBU; ++mb)
            acc[pj][nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mb], b, acc[pj][nb][mb], 0, 0, 0);
        }
    }
  };

  qr_unroll<0, SW - 1>([&](auto I) {
    constexpr int i = decltype(I)::value;
    if constexpr (i < SA - 1) issue_a(std::integral_constant<int, i>{}, i);
    issue_w(std::integral_constant<int, i>{}, i);
  });
  qr_unroll<0, NST>([&](auto C) {
    constexpr int c = decltype(C)::value;
    qr_wait_vm<qr_wait_for(c, SA, SW, NST, nA, nW)>();  // this wave's loads of stage c landed
    qr_wait_lgkm0();  // this wave's reads of stage c - 1 are done before its slots are refilled
    qr_barrier();     // every wave's loads of stage c landed, every read of stage c - 1 done
    if constexpr (c + SA - 1 < NST) issue_a(std::integral_constant<int, (c + SA - 1) % SA>{}, c + SA - 1);
    if constexpr (c + SW - 1 < NST) issue_w(std::integral_constant<int, (c + SW - 1) % SW>{}, c + SW - 1);
    compute(std::integral_constant<int, c % SA>{}, std::integral_constant<int, c % SW>{});
  });

  // lane holds C[4 (lane / 16) + i][lane % 16] of each 16 x 16 block
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const uint32_t col = slice * kCols + wave * NBW * 16u + nb * 16u + lm;
    if (col >= N) continue;
#pragma unroll
    for (int mb = 0; mb < MBU; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t r = mb * 16u + 4u * kb + i;
        if (r >= rows) continue;
        const uint32_t o = (row0 + r) * N + col;  // below 2^32 elements (host checks)
        if constexpr (EPI == kEpiSwiglu) {
          ActBF16::store(p.out, o, swiglu_act<ActBF16>(round_bf16(acc[0][nb][mb][i]), round_bf16(acc[1][nb][mb][i])));
        } else {
          ActBF16::store(p.out, o, round_bf16(acc[0][nb][mb][i]));
        }
      }
  }
}

template <int EPI, int SA, int SW, int NST>
__global__ __launch_bounds__(kQrThreads) void k_qring(GroupedLaunch p) {
  constexpr int PROJ = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int kCols = kQrWRows / PROJ;
  const uint32_t tid = threadIdx.x;
  const uint32_t lin = blockIdx.x;
  const uint32_t slices = (p.n_dim + kCols - 1) / kCols;
  const uint32_t r8 = lin >> 3;
  const uint32_t slice = r8 % slices;
  // XCD x (= lin % 8) takes the x-th eighth of the tiles in order, so the
  // row tiles of one expert follow each other on one XCD
  const uint32_t count = p.tiles != nullptr ? *p.tile_count : (p.rows + kQrTileRows - 1) / kQrTileRows;
  const uint32_t chunk = (count + 7u) / 8u;
  const uint32_t local = r8 / slices;
  if (local >= chunk) return;
  const uint32_t tile = (lin & 7u) * chunk + local;
  if (tile >= count) return;
  // the tile: rows [row0, row0 + rows) of `group`; without a tile list one
  // group (the shared expert) of p.rows rows in order
  uint32_t group, row0, rows;
  if (p.tiles != nullptr) {
    const uint2 td = p.tiles[tile];
    group = td.x;
    row0 = p.row_off[group] + td.y;
    rows = min(p.row_off[group + 1] - row0, static_cast<uint32_t>(kQrTileRows));
  } else {
    group = p.experts;
    row0 = tile * kQrTileRows;
    rows = min(p.rows - row0, static_cast<uint32_t>(kQrTileRows));
  }
  if (rows == 0 || rows > kQrTileRows) return;  // no tile of the sort is empty (and none is longer)
  const uint32_t K = p.k_dim, N = p.n_dim;

  ProjPtrs w[PROJ];
  bool ok = true;
  if (group >= p.experts) {
#pragma unroll
    for (int pj = 0; pj < PROJ; ++pj) w[pj] = p.shared[pj];
    ok = w[0].w != nullptr;
  } else {
    uint32_t index = 0;
    const int kind = resolve_word(group, p.slot_table, p.experts, p.pool, &p.stream, p.dense[0].w != nullptr, index);
    ok = kind != kSrcNone;
#pragma unroll
    for (int pj = 0; pj < PROJ; ++pj) source_proj(kind, index, p.pool, &p.stream, p.dense[pj], p.part[pj], N, K, w[pj]);
  }
  if (!ok) {  // an unresolved expert: its rows are zero (status flagged)
    if (tid == 0 && slice == 0) qr_flag(p.status, 1u);
    for (uint32_t i = tid; i < rows * kCols; i += kQrThreads) {
      const uint32_t r = i / kCols, col = slice * kCols + i % kCols;
      if (col < N) ActBF16::store(p.out, static_cast<size_t>(row0 + r) * N + col, 0.0f);
    }
    return;
  }
#pragma unroll
  for (int pj = 0; pj < PROJ; ++pj) keep_proj(w[pj]);
  // a ring deeper than the stages is cut to them (the short K of a down GEMM)
  constexpr int kSW = SW < NST + 1 ? SW : NST + 1, kSA = SA < kSW ? SA : kSW;
  const uint32_t mbu = (rows + 15u) / 16u;
  if (mbu >= 4) return qr_tile<EPI, 4, kSA, kSW, NST>(p, w, row0, rows, slice);
  if (mbu == 3) return qr_tile<EPI, 3, kSA, kSW, NST>(p, w, row0, rows, slice);
  if (mbu == 2) return qr_tile<EPI, 2, kSA, kSW, NST>(p, w, row0, rows, slice);
  qr_tile<EPI, 1, kSA, kSW, NST>(p, w, row0, rows, slice);
}

template <int EPI, int NST>
hipError_t qring_go(const char* family, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  constexpr int PROJ = EPI == kEpiSwiglu ? 2 : 1;
  constexpr uint32_t kCols = kQrWRows / PROJ;
  const uint32_t slices = (p.n_dim + kCols - 1) / kCols;
  const dim3 grid(slices * ((max_tiles + 7) / 8 * 8));
  auto kernel = &k_qring<EPI, VM_QR_ASLOTS, VM_QR_WSLOTS, NST>;
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events(family, &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, dim3(kQrThreads), 0, stream, start, stop, 0, p);
  else
    hipLaunchKernelGGL(kernel, grid, dim3(kQrThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

// Process-wide choice of the Q4 GEMM of calls above 64 rows: 1 this ring
// kernel, 0 the chunked GEMM of grouped.hip.
static std::atomic<int> g_qring{VM_QRING_DEFAULT};

int qring_mode(int mode) {
  if (mode < 0) return g_qring.load(std::memory_order_relaxed);
  return g_qring.exchange(mode ? 1 : 0, std::memory_order_relaxed);
}

bool qring_supported(int epi, uint32_t k_dim, uint32_t n_dim) {
  if (epi != kEpiSwiglu && epi != kEpiRows) return false;
  return (k_dim == 512 || k_dim == 1024 || k_dim == 2048 || k_dim == 4096) && n_dim > 0 && n_dim % 64 == 0;
}

hipError_t launch_qring(int epi, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  if (!qring_supported(epi, p.k_dim, p.n_dim) || (p.tiles != nullptr) != (p.tile_count != nullptr) ||
      (p.tiles == nullptr && p.rows == 0) || p.a_rows == 0 || static_cast<uint64_t>(p.a_rows) * p.a_stride * 2u > 0xffffffffull ||
      static_cast<uint64_t>(p.n_dim) * p.k_dim > 0xffffffffull)
    return hipErrorInvalidValue;
  const bool own = p.experts == 0;
  const char* family = epi == kEpiSwiglu ? (own ? "shared_gateup" : "grouped_gateup")
                                         : (own ? "shared_down" : "grouped_down");
  switch (p.k_dim) {
    case 512: return epi == kEpiSwiglu ? qring_go<kEpiSwiglu, 4>(family, p, max_tiles, stream)
                                       : qring_go<kEpiRows, 4>(family, p, max_tiles, stream);
    case 1024: return epi == kEpiSwiglu ? qring_go<kEpiSwiglu, 8>(family, p, max_tiles, stream)
                                        : qring_go<kEpiRows, 8>(family, p, max_tiles, stream);
    case 2048: return epi == kEpiSwiglu ? qring_go<kEpiSwiglu, 16>(family, p, max_tiles, stream)
                                        : qring_go<kEpiRows, 16>(family, p, max_tiles, stream);
    default: return epi == kEpiSwiglu ? qring_go<kEpiSwiglu, 32>(family, p, max_tiles, stream)
                                      : qring_go<kEpiRows, 32>(family, p, max_tiles, stream);
  }
}

}  // namespace vm

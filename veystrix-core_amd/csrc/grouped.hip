// Grouped (token-by-expert) kernels of the MoE layer for gfx950: the batched
// decode and chunked prefill path (more than 8 rows).
//
//   sort     count the (token, slot) pairs of every expert with atomics, one
//            block scans the counts into row offsets and a tile list, then the
//            pairs are scattered into expert order (row -> token, pair ->
//            row).  The rows of one expert are contiguous; their order inside
//            the expert changes no result, since every output row is its own
//            set of dot products.  The shared expert is one more group whose
//            rows are all the tokens.
//   gemm     one workgroup per (tile of <= 64 rows of one group, slice of output
//            features).  Workgroups are dealt to the eight XCDs round-robin;
//            each XCD takes a contiguous run of the sorted tiles with all their
//            slices, so the slices of one row tile share its L2 copy of the
//            tile's A rows and the tiles of one expert share its weights.
//            K runs in chunks of eight 32-input groups.  Per chunk the block
//            stages in LDS (one stage for the Q4 GEMMs, two for the router):
//            the A rows (32 lanes per 512-byte row segment, in input order),
//            the Q4 weight row chunks (8 lanes per 128-byte line) and the
//            scale and bias vectors; the 16-byte units of A rows and weight
//            lines are XOR-swizzled so the MFMA lanes' LDS reads are
//            conflict-free.  Each lane dequantises its 16-byte Q4 groups into
//            bf16 in input order
//            (f16 magic number + v_fma_mix + v_cvt_pk_bf16_f32) and feeds
//            v_mfma_f32_16x16x32_bf16 with fp32 accumulation.  The MFMA loop
//            is specialised on the number of 16-row blocks in use, so it has
//            no branch.  Epilogues: SwiGLU of gate and up, bf16 rows (down),
//            router logits (bf16 weights).
//   combine  per token, the expert rows in slot order with the router scores
//            and the shared term.
//
// MFMA operand layout (v_mfma_f32_16x16x32_bf16): lane l supplies 8 bf16 of A
// row l%16 and 8 bf16 of B column l%16, both for the k block l/16; it receives
// C[4*(l/16) + i][l%16], i < 4.  Chunk step st feeds k block kb from group
// g0 + 4*(st/4) + kb, packed word st%4 (8 inputs), so eight steps cover the
// chunk's eight groups and a lane's weight loads are whole 16-byte groups.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kGB = 256;                 // threads per block of the small kernels
constexpr int kCombineSlots = 10;        // top-k bound of the combine (the layer's MAX_TOP_K)
#ifndef VM_GCG
#define VM_GCG 8
#endif
constexpr int kCG = VM_GCG;              // 32-input groups per K chunk (8: a 128-byte line per weight row)
// A chunk's scale and bias vectors are staged with one 16-byte load of eight
// groups from the chunk's first group, and full (non-tail) kernels need K to be
// a multiple of the chunk: any other chunk size would read past the row.
static_assert(kCG == 8, "the scale and bias staging covers exactly eight groups per chunk");
constexpr int kHalves = kCG / 4;         // groups per lane and chunk
constexpr int kSteps = 4 * kHalves;      // MFMA k steps per chunk

// LDS layouts of the staged A rows and weight lines.  A wave64 ds_read_b128
// serves 16 lanes per cycle from 64 four-byte banks, and the lanes it serves
// together are not 16 consecutive ones: a row padding of 16 bytes (the usual
// remedy) left both the MFMA A reads (lane = row am, k block akb) and the
// weight-line reads (lane = column bn, group bkb) two-way conflicted, 8.2
// cycles per wave read instead of 4.5 in a timing of each read pattern.
// XORing the 16-byte unit index with bits of the row (column) makes every
// read step of both loops conflict-free in the same timing and needs no
// padding.  A row r stores its logical unit u at unit u ^ a_swz(r); the
// swizzle depends on r mod 16 only, the row within an MFMA block.  The XOR
// reaches the step bits of the unit, so each read step needs an address of
// its own: in the down GEMM the extra registers cost its second block per CU
// (40 % slower), so its rows keep the padded layout, whose step offsets are
// immediates.
template <int EPI>
constexpr bool swz_rows() { return EPI != kEpiRows; }
// LDS bytes per staged A row
template <int EPI>
constexpr int row_bytes() { return swz_rows<EPI>() ? kCG * 64 : kCG * 64 + 16; }
__device__ __forceinline__ constexpr uint32_t a_swz(uint32_t r) { return (r & 3u) | ((r & 12u) << 1); }
// A weight line of column c stores its group g at unit g ^ w_swz(c).
__device__ __forceinline__ constexpr uint32_t w_swz(uint32_t c) { return c & 7u; }

// Bytes of one LDS stage of a grouped GEMM instance: the A rows, then for Q4
// weights without a tail chunk the chunk's scale and bias vectors of every
// column of the block (16 bytes each).
#ifndef VM_LDS_B
#define VM_LDS_B 1
#endif
// the down GEMM (K = the intermediate size, two chunks) stages its weights too:
// with one LDS stage (grouped_tile) two blocks still fit per CU, and the
// coalesced line loads beat loads straight into the MFMA lanes (2048 rows
// 124 -> 119 us, 8192 rows 377 -> 364 us)
#ifndef VM_LDS_B_DN
#define VM_LDS_B_DN 1
#endif
constexpr int kWColBytes = kCG * 16;  // LDS bytes per staged weight row chunk (unpadded: the groups are swizzled)

// Q4 weights staged through LDS (coalesced 128-byte row loads by the whole
// block) rather than loaded by the MFMA lanes themselves.
template <int EPI, bool TAIL>
constexpr bool lds_weights() {
  return (EPI == kEpiRows ? VM_LDS_B_DN : VM_LDS_B) && EPI != kEpiLogits && !TAIL;
}

// Rows per tile of a grouped GEMM instance.
template <int EPI>
constexpr int tile_rows() {
  return EPI == kEpiRows ? kGroupedRowsDown : EPI == kEpiLogits ? kGroupedRowsRouter : kGroupedRows;
}

template <int EPI, int WAVES, int NBW, int PROJ, bool TAIL, int TR = tile_rows<EPI>()>
constexpr int stage_bytes() {
  return TR * row_bytes<EPI>() + (EPI != kEpiLogits && !TAIL ? PROJ * 2 * WAVES * NBW * 16 * 16 : 0) +
         (lds_weights<EPI, TAIL>() ? PROJ * WAVES * NBW * 16 * kWColBytes : 0);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ uint4 g_zero_page[64];  // lanes without data load zeros from here

__device__ __forceinline__ void flag(uint32_t* status, uint32_t bits) {
  if (status != nullptr) atomicOr(status, bits);
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// f16 magic for the nibble decode, kept in a VGPR so that every decode is one
// v_and_or_b32 (a literal mask and a register magic).
__device__ __forceinline__ uint32_t f16_magic() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}

// Operand order of the MFMA k slots: 1 = input order (the activation rows
// are used as loaded and the dequantised pairs are packed (q_0 q_1) .. (q_6
// q_7)); 0 = pair-permuted ((q_n q_{n+4}) pairs, with every activation unit
// permuted the same way when it is staged).  Both feed each k slot the same
// product; the MFMA's sum does not depend on the slot order (the two give the
// same bits).
#ifndef VM_DQ_NATURAL
#define VM_DQ_NATURAL 1
#endif
constexpr bool kNatural = VM_DQ_NATURAL;

// 8 inputs of one packed word -> 4 bf16 pairs in the operand order above.
// (1024 + q) and (1024 + 16 q) are exact in f16, so w = s*q + b is one fp32
// fma per value: s*(1024 + q) + (b - 1024 s) for the low nibble of a byte
// and (s/16)*(1024 + 16 q) + (b - 64 s) for the high one.
struct Dequant {
  float s, b1024, s16, b64;
  __device__ __forceinline__ Dequant(float scale, float b) {
    s = scale;
    b1024 = fmaf(-1024.0f, s, b);
    s16 = 0.0625f * s;
    b64 = fmaf(-64.0f, s, b);
  }
  // EAGER: each pair is packed as soon as it is computed.  The down GEMM
  // needs it: computing all eight values first held two more VGPRs there
  // (130), which cost it its second block per CU (2048 rows 125 -> 106 us
  // with it).  The gate/up GEMM and the 16-row kernels run faster with the
  // eight values computed first (2048-row gate/up 200.5 -> 195.5 us).
  template <bool EAGER = false>
  __device__ __forceinline__ void word(uint32_t w, uint32_t magic, uint32_t out[4]) const {
    const uint32_t w8 = w >> 8;
    const uint32_t m[4] = {(w & 0x000F000Fu) | magic, (w & 0x00F000F0u) | magic, (w8 & 0x000F000Fu) | magic,
                           (w8 & 0x00F000F0u) | magic};
    const f16x2_t h[4] = {__builtin_bit_cast(f16x2_t, m[0]), __builtin_bit_cast(f16x2_t, m[1]),
                          __builtin_bit_cast(f16x2_t, m[2]), __builtin_bit_cast(f16x2_t, m[3])};
    // q_n from h[n].x and q_{n+4} from h[n].y, n < 4 (odd n: the high nibble of a byte)
    auto q = [&](int n, bool high) {
      const float sc = n & 1 ? s16 : s, bc = n & 1 ? b64 : b1024;
      return fmaf(sc, static_cast<float>(high ? h[n].y : h[n].x), bc);
    };
    if constexpr (EAGER) {
      if constexpr (kNatural) {
        out[0] = pack_bf16(q(0, false), q(1, false));
        out[2] = pack_bf16(q(0, true), q(1, true));
        out[1] = pack_bf16(q(2, false), q(3, false));
        out[3] = pack_bf16(q(2, true), q(3, true));
      } else {
#pragma unroll
        for (int n = 0; n < 4; ++n) out[n] = pack_bf16(q(n, false), q(n, true));
      }
      return;
    }
    float lo[4], hi[4];  // q_n and q_{n+4}, n < 4
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      lo[n] = q(n, false);
      hi[n] = q(n, true);
    }
    if constexpr (kNatural) {
      out[0] = pack_bf16(lo[0], lo[1]);
      out[1] = pack_bf16(lo[2], lo[3]);
      out[2] = pack_bf16(hi[0], hi[1]);
      out[3] = pack_bf16(hi[2], hi[3]);
    } else {
#pragma unroll
      for (int n = 0; n < 4; ++n) out[n] = pack_bf16(lo[n], hi[n]);
    }
  }
};

// bf16 weights in the operand order: as loaded, or natural pairs (k0 k1)(k2
// k3)(k4 k5)(k6 k7) -> (k0 k4)(k1 k5)(k2 k6)(k3 k7)
__device__ __forceinline__ void permute_word(const uint4 v, uint32_t out[4]) {
  if constexpr (kNatural) {
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  } else {
    out[0] = (v.x & 0xffffu) | (v.z << 16);
    out[1] = (v.x >> 16) | (v.z & 0xffff0000u);
    out[2] = (v.y & 0xffffu) | (v.w << 16);
    out[3] = (v.y >> 16) | (v.w & 0xffff0000u);
  }
}

__device__ __forceinline__ bf16x8_t as_operand(const uint32_t r[4]) {
  const uint4 v = make_uint4(r[0], r[1], r[2], r[3]);
  return __builtin_bit_cast(bf16x8_t, v);
}

// ------------------------------------------------------------------ gemm ---

// B side of one lane for one chunk: groups g0 + 4 h + kb (h < kHalves) of
// one weight row, Q4 (16 bytes + scale + bias each) or bf16 (32 weights each).
// Chunk step st uses half st/4, packed word st%4.
template <bool Q4, bool TAIL>
struct BChunk;

// Q4, full chunk: the weights only.  The chunk's scales and biases are
// staged in LDS with the activations (one 16-byte load per row for the whole
// block, pair-permuted so that lane kb finds its groups kb and 4 + kb in one
// dword each) and come into step() as bf16 pairs.
template <>
struct BChunk<true, false> {
  uint4 w[kHalves];
  __device__ __forceinline__ void load(const ProjPtrs& p, uint32_t wrow, uint32_t, uint32_t g0, uint32_t kb,
                                       uint32_t, bool) {
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(p.w) + g0 * 16u;
    const uint32_t wl = wrow + kb * 16u;
#pragma unroll
    for (int h = 0; h < kHalves; ++h) w[h] = ldg16(wb + wl + h * 64u);
  }
  // s2/b2: the scales/biases of groups kb (low half) and 4 + kb (high half)
  template <bool EAGER>
  __device__ __forceinline__ bf16x8_t step(int st, uint32_t magic, uint32_t s2, uint32_t b2) const {
    const int h = st >> 2, i = st & 3;
    const float sc = __uint_as_float(h ? s2 & 0xffff0000u : s2 << 16);
    const float bi = __uint_as_float(h ? b2 & 0xffff0000u : b2 << 16);
    const Dequant dq(sc, bi);
    const uint32_t word = i == 0 ? w[h].x : i == 1 ? w[h].y : i == 2 ? w[h].z : w[h].w;
    uint32_t r[4];
    dq.template word<EAGER>(word, magic, r);
    return as_operand(r);
  }
};

// Q4, tail chunk: groups past the end are clamped (their activations are
// staged as zeros); scales and biases one by one.
template <>
struct BChunk<true, true> {
  uint4 w[kHalves];
  uint32_t s[kHalves], b[kHalves];
  __device__ __forceinline__ void load(const ProjPtrs& p, uint32_t wrow, uint32_t mrow, uint32_t g0, uint32_t kb,
                                       uint32_t G, bool) {
#pragma unroll
    for (int h = 0; h < kHalves; ++h) {
      const uint32_t g = min(g0 + 4 * h + kb, G - 1);
      w[h] = ldg16(reinterpret_cast<const uint8_t*>(p.w) + wrow + g * 16u);
      s[h] = ldg_u16(reinterpret_cast<const uint8_t*>(p.s) + mrow + g * 2u);
      b[h] = ldg_u16(reinterpret_cast<const uint8_t*>(p.b) + mrow + g * 2u);
    }
  }
  template <bool EAGER>
  __device__ __forceinline__ bf16x8_t step(int st, uint32_t magic, uint32_t, uint32_t) const {
    const int h = st >> 2, i = st & 3;
    const Dequant dq(bf16_to_f32(s[h]), bf16_to_f32(b[h]));
    const uint32_t word = i == 0 ? w[h].x : i == 1 ? w[h].y : i == 2 ? w[h].z : w[h].w;
    uint32_t r[4];
    dq.template word<EAGER>(word, magic, r);
    return as_operand(r);
  }
};

template <bool TAIL>
struct BChunk<false, TAIL> {
  uint4 v[kHalves][4];
  // router: bf16 weights [N, K]; wrow = byte offset of the row
  __device__ __forceinline__ void load(const uint16_t* wbf, uint32_t wrow, uint32_t, uint32_t g0, uint32_t kb,
                                       uint32_t G, bool tail) {
#pragma unroll
    for (int h = 0; h < kHalves; ++h) {
      const uint32_t g = tail ? min(g0 + 4 * h + kb, G - 1) : g0 + 4 * h + kb;
      const uint8_t* src = reinterpret_cast<const uint8_t*>(wbf) + wrow + g * 64u;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[h][i] = ldg16(src + 16 * i);
    }
  }
  template <bool EAGER>
  __device__ __forceinline__ bf16x8_t step(int st, uint32_t, uint32_t, uint32_t) const {
    uint32_t r[4];
    permute_word(v[st >> 2][st & 3], r);
    return as_operand(r);
  }
};

// Column slices per block of the one-stage GEMMs (a power of two; the
// launch halves it until it divides the call's slices).  The down GEMM's
// blocks are short (two K chunks), so their fixed part (tile lookups, the
// first chunk's loads, the epilogue) weighed half of each block; with two
// slices per block the second slice's first loads overlap the first's last
// chunk.  The gate/up GEMM keeps one: the loop state that the epilogue then
// keeps live costs its third block per CU (176 VGPRs).
#ifndef VM_GU_SPB
#define VM_GU_SPB 1
#endif
#ifndef VM_DN_SPB
#define VM_DN_SPB 2
#endif
template <int EPI>
constexpr uint32_t slices_per_block() {
  return EPI == kEpiSwiglu ? VM_GU_SPB : EPI == kEpiRows ? VM_DN_SPB : 1;
}

// The tile body for MBU 16-row blocks in use (rows <= 16 * MBU): the A
// staging covers those rows only and the MFMA loops carry no branch, so the
// LDS reads of a step and the MFMAs of neighbouring steps can be scheduled
// freely.
template <int EPI, int WAVES, int NBW, int PROJ, bool TAIL, int MBU, bool WNT, int TR>
__device__ __forceinline__ void grouped_tile(const GroupedLaunch& p, const ProjPtrs (&w)[PROJ], uint32_t row0,
                                             uint32_t rows, uint32_t slice0, uint32_t nslices, uint8_t* s_a0) {
  constexpr bool Q4 = EPI != kEpiLogits;
  constexpr int kThreads = WAVES * 64;
  constexpr int kUnits = kCG * 4;                                // 16-byte A units per row and chunk
  constexpr int kItemsAll = MBU * 16 * kUnits;                  // A units per stage
  constexpr int kItems = (kItemsAll + kThreads - 1) / kThreads;  // per thread
  constexpr bool kAllItems = kItemsAll % kThreads == 0;

  constexpr bool kSwz = swz_rows<EPI>();
  constexpr int kRowB = row_bytes<EPI>();
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t K = p.k_dim, N = p.n_dim, G = K / kGroup;
  uint32_t slice = slice0;  // the slice being computed (the weights' offsets may already be the next one's)
  const uint32_t n_wave = (slice0 * WAVES + wave) * NBW * 16;  // B lanes of the two-stage path (one slice)

  // A staging: unit it = tid + j * threads -> (row it / kUnits, 16-byte unit
  // it % kUnits of the chunk): 32 consecutive lanes read one row's 512
  // contiguous bytes, so a wave's load covers whole cache lines.  Rows past
  // the tile repeat its first row: an MFMA output row depends on its own A
  // row only, and those rows are not stored.  Every global load of the loop
  // is a wave-uniform base (SGPRs, advanced per chunk by scalar adds) plus a
  // 32-bit byte offset per lane: one VGPR per address and no 64-bit address
  // arithmetic per chunk (launch_grouped keeps the A matrix under 4 GiB).
  static_assert(kThreads % kUnits == 0, "an item step covers whole rows");
  constexpr int kRS = kThreads / kUnits;  // rows per item step
  const uint32_t a_u = tid % kUnits;      // the thread's 16-byte unit, the same for every item
  uint32_t a_vo[kItems];
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const uint32_t r = tid / kUnits + kRS * j;
    const uint32_t rr = r < rows ? r : 0u;
    const uint32_t arow = p.row_token != nullptr ? p.row_token[row0 + rr] : row0 + rr;
    a_vo[j] = (arow * p.a_stride + a_u * 8) * 2u;
  }
  // LDS offset of item j: the swizzle depends on the row mod 16, so it
  // repeats every kP items and the rest of the offset is an immediate
  constexpr int kP = !kSwz || kRS % 16 == 0 ? 1 : kRS % 8 == 0 ? 2 : kRS % 4 == 0 ? 4 : kRS % 2 == 0 ? 8 : 16;
  constexpr int kPA = kP < kItems ? kP : kItems;
  uint32_t a_off0[kPA];
#pragma unroll
  for (int j = 0; j < kPA; ++j) {
    const uint32_t r = tid / kUnits + kRS * j;
    a_off0[j] = r * kRowB + (a_u ^ (kSwz ? a_swz(r) : 0u)) * 16;
  }
  auto a_off = [&](int j) { return a_off0[j % kPA] + (j / kPA) * (kPA * kRS * kRowB); };
  // scale staging (Q4, full chunks): vector v = tid + j * threads -> (proj,
  // scales or biases, column of the block); 16 bytes = the chunk's 8 groups
  constexpr int kCols = WAVES * NBW * 16;
  constexpr bool kLdsScales = Q4 && !TAIL;
  constexpr int kSVecs = kLdsScales ? PROJ * 2 * kCols : 0;
  constexpr int kSItems = (kSVecs + kThreads - 1) / kThreads;
  constexpr int kStage = stage_bytes<EPI, WAVES, NBW, PROJ, TAIL, TR>();
  constexpr int kStageBytes = TR * kRowB;  // the A rows of a stage
  const uint8_t* sv_base[kSItems > 0 ? kSItems : 1];  // wave-uniform
  uint32_t sv_vo[kSItems > 0 ? kSItems : 1];
#pragma unroll
  for (int j = 0; j < kSItems; ++j) {
    static_assert(kCols % 64 == 0, "a wave's vectors share one (projection, scales or biases)");
    const uint32_t v = min(tid + j * kThreads, static_cast<uint32_t>(kSVecs - 1));
    // (projection, scales or biases) is wave-uniform: select it in SGPRs (an
    // indexed private array of pointers would go to scratch)
    const uint32_t q = __builtin_amdgcn_readfirstlane(v / kCols);
    const uint32_t col = min(slice0 * kCols + v % kCols, N - 1);
    const uint16_t *ps0 = w[0].s, *pb0 = w[0].b, *ps1 = w[PROJ - 1].s, *pb1 = w[PROJ - 1].b;
    VM_KEEP(ps0);  // opaque copies: a select of loads from `w` would become an indexed load
    VM_KEEP(pb0);
    VM_KEEP(ps1);
    VM_KEEP(pb1);
    sv_base[j] = reinterpret_cast<const uint8_t*>(q >= 2 ? ((q & 1u) ? pb1 : ps1) : ((q & 1u) ? pb0 : ps0));
    sv_vo[j] = col * G * 2u;
  }
  // weight staging (lds_weights): item it = tid + j * threads -> (projection,
  // column of the block, group of the chunk); eight lanes read one row's
  // 128-byte chunk line.  The projection is the same for all items of one j.
  constexpr bool kLdsB = lds_weights<EPI, TAIL>();
  constexpr int kWVecs = kLdsB ? PROJ * kCols * kCG : 0;
  constexpr int kWItems = kWVecs / kThreads;
  constexpr int kWArea = kStageBytes + (kLdsScales ? PROJ * 2 * kCols * 16 : 0);
  static_assert(!kLdsB || (kWVecs % kThreads == 0 && (kCols * kCG) % kThreads == 0), "whole items per thread");
  uint32_t w_vo[kWItems > 0 ? kWItems : 1];  // byte offsets from the projection's weights
  uint32_t w_off[kWItems > 0 ? kWItems : 1];
#pragma unroll
  for (int j = 0; j < kWItems; ++j) {
    constexpr int kPerProj = kCols * kCG;
    const uint32_t it = tid + j * kThreads;
    const uint32_t ci = (it % kPerProj) / kCG, g = it % kCG;
    const uint32_t col = min(slice0 * kCols + ci, N - 1);
    w_vo[j] = col * (K / 2) + g * 16u;
    w_off[j] = kWArea + ((j * kThreads) / kPerProj * kCols + ci) * kWColBytes + (g ^ w_swz(ci)) * 16u;
  }
  // the weight and scale offsets move on to the next slice (the A rows stay);
  // blocks of several slices have N a multiple of the block's columns, so no
  // column is clamped
  auto next_slice = [&]() {
#pragma unroll
    for (int j = 0; j < kSItems; ++j) sv_vo[j] += kCols * G * 2u;
#pragma unroll
    for (int j = 0; j < kWItems; ++j) w_vo[j] += kCols * (K / 2);
  };
  uint4 ar[kItems], sr[kSItems > 0 ? kSItems : 1], wr[kWItems > 0 ? kWItems : 1];
  // The offsets pass through an empty asm so that loop strength reduction
  // does not turn them back into one 64-bit pointer per load.
  auto opaque = [](uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
  };
  auto a_load = [&](uint32_t g0, bool tail) {
    const uint8_t* ab = reinterpret_cast<const uint8_t*>(p.a) + g0 * (kGroup * 2u);
    const bool zero = tail && g0 + a_u / 4 >= G;  // the thread's unit is past K
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      if (!kAllItems && tid + j * kThreads >= static_cast<uint32_t>(kItemsAll)) continue;
      ar[j] = ldg16(TAIL && zero ? reinterpret_cast<const uint8_t*>(g_zero_page) : ab + opaque(a_vo[j]));
    }
#pragma unroll
    for (int j = 0; j < kSItems; ++j) sr[j] = ldg16(sv_base[j] + g0 * 2u + opaque(sv_vo[j]));
#pragma unroll
    for (int j = 0; j < kWItems; ++j) {
      constexpr int kPerProj = kCols * kCG;
      const int pj = (j * kThreads) / kPerProj;  // compile-time
      const uint8_t* src = reinterpret_cast<const uint8_t*>(w[pj].w) + g0 * 16u + opaque(w_vo[j]);
      wr[j] = WNT ? ldg16_nt(src) : ldg16(src);
    }
  };
  // (x0 x1)(x2 x3)(x4 x5)(x6 x7) -> (x0 x4)(x1 x5)(x2 x6)(x3 x7)
  auto pair_perm = [](const uint4 v) {
    return make_uint4((v.x & 0xffffu) | (v.z << 16), (v.x >> 16) | (v.z & 0xffff0000u),
                      (v.y & 0xffffu) | (v.w << 16), (v.y >> 16) | (v.w & 0xffff0000u));
  };
  auto a_store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      if (!kAllItems && tid + j * kThreads >= static_cast<uint32_t>(kItemsAll)) continue;
      *reinterpret_cast<uint4*>(s_a0 + buf * kStage + a_off(j)) = kNatural ? ar[j] : pair_perm(ar[j]);
    }
#pragma unroll
    for (int j = 0; j < kSItems; ++j) {
      if (kSVecs % kThreads != 0 && tid + j * kThreads >= static_cast<uint32_t>(kSVecs)) continue;
      *reinterpret_cast<uint4*>(s_a0 + buf * kStage + kStageBytes + (tid + j * kThreads) * 16) = pair_perm(sr[j]);
    }
#pragma unroll
    for (int j = 0; j < kWItems; ++j) *reinterpret_cast<uint4*>(s_a0 + buf * kStage + w_off[j]) = wr[j];
  };

  // B: lane -> (column lane%16 of each block, group g0 + lane/16); columns
  // past N read the last row and are not stored
  const uint32_t bn = lane & 15u, bkb = lane >> 4;
  uint32_t wrow[NBW], mrow[NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const uint32_t col = min(n_wave + nb * 16 + bn, N - 1);
    wrow[nb] = Q4 ? col * (K / 2) : col * K * 2;
    mrow[nb] = col * G * 2;
  }
  BChunk<Q4, TAIL> b0[PROJ][NBW], b1[PROJ][NBW];
  auto b_load = [&](BChunk<Q4, TAIL> (&dst)[PROJ][NBW], uint32_t g0, bool tail) {
#pragma unroll
    for (int pj = 0; pj < PROJ; ++pj) {
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        if constexpr (Q4) dst[pj][nb].load(w[pj], wrow[nb], mrow[nb], g0, bkb, G, tail);
        else dst[pj][nb].load(p.bf16_weight, wrow[nb], 0u, g0, bkb, G, tail);
      }
    }
  };

  f32x4_t acc[PROJ][NBW][MBU];
#pragma unroll
  for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
      for (int mb = 0; mb < MBU; ++mb) acc[pj][nb][mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t chunks = (G + kCG - 1) / kCG;
  const uint32_t magic = Q4 ? f16_magic() : 0u;
  const uint32_t am = lane & 15u, akb = lane >> 4;
  // the lane's unit of step st is (16 (st / 4) + 4 akb + st % 4) ^ a_swz(am);
  // the three terms occupy disjoint bits, so the step's part is XORed on last
  const uint32_t a_lane = am * kRowB + ((akb * 4) ^ (kSwz ? a_swz(am) : 0u)) * 16;
  const uint32_t w_lane = (bkb ^ w_swz(bn)) * 16;  // the group part of the weight-line reads
  // The gate/up waves raise their issue priority (s_setprio, a wave's own
  // scheduling priority on its SIMD) while they compute a chunk.  Three blocks
  // share a CU, each in its own phase; with the raise the SIMD prefers the
  // waves whose dequantisation and MFMAs are ready over those of a block that
  // is issuing its next loads or storing them to LDS.  Same instructions, same
  // bits; on three boxes the 2048-row gate/up took 193.5-208.9 -> 191.5-201.5
  // us and the 8192-row window's 503-545 -> 488-527 us.  The raise during the
  // LDS-store phase instead, a higher level (2 or 3), or the same raise in the
  // down GEMM gained nothing consistent.
  constexpr bool kPrio = EPI == kEpiSwiglu;
  auto compute = [&](int buf, const BChunk<Q4, TAIL> (&bc)[PROJ][NBW]) {
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
    const uint8_t* s_a = s_a0 + buf * kStage;
    BChunk<Q4, TAIL> bl[PROJ][NBW];
    uint32_t s2[PROJ][NBW], b2[PROJ][NBW];
#pragma unroll
    for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb) {
        s2[pj][nb] = b2[pj][nb] = 0;
        if constexpr (kLdsScales) {
          const uint32_t col = wave * NBW * 16 + nb * 16 + bn;
          const uint32_t* sv = reinterpret_cast<const uint32_t*>(s_a0 + buf * kStage + kStageBytes);
          s2[pj][nb] = sv[((pj * 2 + 0) * kCols + col) * 4 + bkb];
          b2[pj][nb] = sv[((pj * 2 + 1) * kCols + col) * 4 + bkb];
        }
      }
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const uint32_t a_step = (st >> 2) * 256u + (st & 3) * 16u;
      bf16x8_t aop[MBU];
#pragma unroll
      for (int mb = 0; mb < MBU; ++mb)
        aop[mb] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(
                                                   s_a + mb * 16 * kRowB + (kSwz ? a_lane ^ a_step : a_lane + a_step)));
      if constexpr (kLdsB) {
        if ((st & 3) == 0) {  // the lane's group 4 h + kb of each of its rows, from LDS
#pragma unroll
          for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
            for (int nb = 0; nb < NBW; ++nb) {
              const uint32_t col = wave * NBW * 16 + nb * 16 + bn;
              bl[pj][nb].w[st >> 2] = *reinterpret_cast<const uint4*>(
                  s_a0 + buf * kStage + kWArea + (pj * kCols + col) * kWColBytes + (w_lane ^ ((st >> 2) * 64u)));
            }
        }
      }
#pragma unroll
      for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
          // the down GEMM packs each dequantised pair as it is computed
          constexpr bool kEager = EPI == kEpiRows;
          const bf16x8_t bop = kLdsB ? bl[pj][nb].template step<kEager>(st, magic, s2[pj][nb], b2[pj][nb])
                                     : bc[pj][nb].template step<kEager>(st, magic, s2[pj][nb], b2[pj][nb]);
#pragma unroll
          for (int mb = 0; mb < MBU; ++mb)
            acc[pj][nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[mb], bop, acc[pj][nb][mb], 0, 0, 0);
        }
    }
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
  };
  // only a K that is not a multiple of the chunk has a tail chunk
  auto tail_chunk = [&](uint32_t c) { return TAIL && (c + 1) * kCG > G; };
  // epilogue of slice s: lane holds rows 4*(lane/16) + i of every row block, column lane%16
  auto epilogue = [&](uint32_t s) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      const uint32_t col = (s * WAVES + wave) * NBW * 16 + nb * 16 + bn;
      if (col >= N) continue;
#pragma unroll
      for (int mb = 0; mb < MBU; ++mb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t r = mb * 16 + 4 * bkb + i;
          if (r >= rows) continue;
          const uint32_t o = (row0 + r) * N + col;  // outputs stay below 2^32 elements (host checks)
          if constexpr (EPI == kEpiSwiglu) {
            const float gv = round_bf16(acc[0][nb][mb][i]);
            const float uv = round_bf16(acc[PROJ - 1][nb][mb][i]);
            ActBF16::store(p.out, o, swiglu_act<ActBF16>(gv, uv));
          } else if constexpr (EPI == kEpiRows) {
            ActBF16::store(p.out, o, round_bf16(acc[0][nb][mb][i]));
          } else {
            float v = acc[0][nb][mb][i];
            if (p.bias != nullptr) v += p.bias[col];
            static_cast<float*>(p.out)[o] = round_bf16(v);
          }
        }
      }
    }
  };

  // Loads run one chunk ahead.  With staged weights (gate/up, down) there is one
  // LDS stage: the next chunk waits in registers while this one is computed
  // and a second barrier guards its store.  Half the LDS of a double buffer
  // lets several 4-wave blocks share a CU, whose barriers then do not hold
  // each other up (gate/up at 2048 rows 258 -> 237 us against one 8-wave
  // block with two stages; 700 -> 651 us at 8192; with the 32-bit load
  // offsets three blocks fit, 232 -> 208 us and 660 -> 586 us).  Without
  // staged weights (the router, tail chunks) the two-stage ping-pong stays:
  // the copy of the next chunk's B registers makes the end of a chunk wait for
  // them; an unrolled ping-pong without that wait, and a third register set,
  // both measured slower.
  if constexpr (kLdsB) {
    // The block's slices run back to back: during the last chunk of a slice
    // the first chunk of the next one loads (same A rows, the next columns'
    // weights), so the next slice starts without the load latency and the
    // epilogue's stores overlap the loads.
    a_load(0, tail_chunk(0));
    a_store(0);
    __syncthreads();
    if constexpr (slices_per_block<EPI>() == 1) {
      // one slice: the epilogue after the loop, where the loop's offsets are dead
      for (uint32_t c = 0; c < chunks; ++c) {
        const bool more = c + 1 < chunks;
        if (more) a_load((c + 1) * kCG, tail_chunk(c + 1));
        compute(0, b0);
        __syncthreads();
        if (more) {
          a_store(0);
          __syncthreads();
        }
      }
      epilogue(slice0);
      return;
    }
    for (uint32_t k = 0; k < nslices; ++k) {
      for (uint32_t c = 0; c < chunks; ++c) {
        const bool more = c + 1 < chunks || k + 1 < nslices;
        if (c + 1 < chunks) {
          a_load((c + 1) * kCG, tail_chunk(c + 1));
        } else if (more) {
          next_slice();
          a_load(0, tail_chunk(0));
        }
        compute(0, b0);
        __syncthreads();
        if (more) {
          a_store(0);
          __syncthreads();
        }
        if (c + 1 == chunks) {  // after the store: the prefetch registers are free for the epilogue
          epilogue(slice);
#pragma unroll
          for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
            for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
              for (int mb = 0; mb < MBU; ++mb) acc[pj][nb][mb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
          ++slice;
        }
      }
    }
  } else {
    a_load(0, tail_chunk(0));
    b_load(b0, 0, tail_chunk(0));
    a_store(0);
    __syncthreads();
    for (uint32_t c = 0; c < chunks; ++c) {
      const int buf = c & 1;
      const bool more = c + 1 < chunks;
      if (more) {
        a_load((c + 1) * kCG, tail_chunk(c + 1));
        b_load(b1, (c + 1) * kCG, tail_chunk(c + 1));
      }
      compute(buf, b0);
      if (more) {
        a_store(buf ^ 1);
#pragma unroll
        for (int pj = 0; pj < PROJ; ++pj)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb) b0[pj][nb] = b1[pj][nb];
      }
      __syncthreads();
    }
    epilogue(slice0);
  }
}

template <int EPI, int WAVES, int NBW, int PROJ, bool TAIL, bool WNT, int TR>
__device__ __forceinline__ void grouped_block(const GroupedLaunch& p, uint32_t lin, uint8_t* s_a0);

// EPI: 0 SwiGLU of projections 0 (gate) and 1 (up) -> bf16 [rows, N];
//      1 bf16 rows -> [rows, N]; 2 router logits (bf16 weights) -> fp32 [rows, N].
// TAIL: K is not a multiple of the chunk (kCG groups); the last chunk clamps.
#ifndef VM_G_WAVES_PER_EU
#define VM_G_WAVES_PER_EU 1
#endif
// The down GEMM runs two 8-wave blocks per CU (its LDS allows two): four waves
// per SIMD, so its VGPRs must stay at or below 128.  Above that only one block
// fits and the kernel takes 40 % longer.
#ifndef VM_DN_WAVES_PER_EU
#define VM_DN_WAVES_PER_EU 2
#endif
// Block order of sorted tiles: 0 deals row tiles to the XCDs round-robin
// (tile t on XCD t % 8); 1 gives each XCD a contiguous run of the tiles, so
// the row tiles of one expert share that XCD's L2 copy of its weights.
#ifndef VM_G_MAP
#define VM_G_MAP 1
#endif
// WNT: the weight lines are loaded non-temporal, for calls whose experts
// mostly hold one row tile (each line is read once; kept from the L2 they
// displaced the tile's activation rows, which the column slices share: the
// 2048-row gate/up fetched 28 % above its bytes).  Calls with several row
// tiles per expert keep cached loads (the tiles of an expert share its
// weights in the L2; non-temporal loads there cost 5 %).
template <int EPI, int WAVES, int NBW, int PROJ, bool TAIL, bool WNT, int TR>
__global__ __launch_bounds__(WAVES * 64)
__attribute__((amdgpu_waves_per_eu(EPI == kEpiRows ? VM_DN_WAVES_PER_EU : VM_G_WAVES_PER_EU)))
void k_grouped(GroupedLaunch p) {
  static_assert(TR % 16 == 0 && TR <= 96, "tiles are one to six 16-row blocks");
  extern __shared__ uint4 s_dyn[];  // two stages of stage_bytes<...>()
  uint8_t* s_a0 = reinterpret_cast<uint8_t*>(s_dyn);
  const uint32_t tid = threadIdx.x;

  // XCD-aware order: workgroups are dealt to the eight XCDs round-robin, so
  // block L runs on XCD L % 8.  The column slices of one row tile take
  // consecutive blocks of the same XCD and share its L2 copy of the tile's A
  // rows.  Sorted tiles: XCD x takes the x-th eighth of the tiles in order,
  // so the row tiles of one expert also follow each other on one XCD and
  // share its weights.  A block computes p.spb consecutive slices of its
  // tile (see grouped_tile).  The grid is slices / spb * (tile bound rounded
  // up to a multiple of 8); blocks past the live tile count exit.
  if constexpr (EPI == kEpiLogits) {
    if (blockIdx.x == 0 && p.zero_words != nullptr)
      for (uint32_t i = tid; i < p.zero_count; i += WAVES * 64) p.zero_words[i] = 0;
  }
  grouped_block<EPI, WAVES, NBW, PROJ, TAIL, WNT, TR>(p, blockIdx.x, s_a0);
}

// One block's work item `lin` (the XCD-aware order of k_grouped).
template <int EPI, int WAVES, int NBW, int PROJ, bool TAIL, bool WNT, int TR>
__device__ __forceinline__ void grouped_block(const GroupedLaunch& p, uint32_t lin, uint8_t* s_a0) {
  constexpr int kBM = TR;
  constexpr int kMB = kBM / 16;  // MFMA row blocks
  constexpr bool Q4 = EPI != kEpiLogits;
  const uint32_t tid = threadIdx.x;
  const uint32_t slices = (p.n_dim + WAVES * NBW * 16 - 1) / (WAVES * NBW * 16);
  const uint32_t nslices = p.spb, sgroups = slices / nslices;
  const uint32_t r8 = lin >> 3;
  const uint32_t slice0 = (r8 % sgroups) * nslices;
  uint32_t tile = (r8 / sgroups) * 8 + (lin & 7u);
#if VM_G_MAP == 1
  if (p.tiles != nullptr) {
    const uint32_t chunk = (*p.tile_count + 7u) / 8u;
    const uint32_t local = r8 / sgroups;
    if (local >= chunk) return;
    tile = (lin & 7u) * chunk + local;
  }
#endif

  // the tile: rows [row0, row0 + rows) of `group`
  uint32_t group = 0, row0, rows;
  if (p.tiles != nullptr) {
    if (tile >= *p.tile_count) return;
    const uint2 td = p.tiles[tile];
    group = td.x;
    row0 = p.row_off[group] + td.y;
    rows = min(p.row_off[group + 1] - row0, static_cast<uint32_t>(kBM));
  } else {
    row0 = tile * kBM;
    if (row0 >= p.rows) return;
    rows = min(p.rows - row0, static_cast<uint32_t>(kBM));
  }
  const uint32_t K = p.k_dim, N = p.n_dim;

  // the group's weights
  ProjPtrs w[PROJ];
  if constexpr (Q4) {
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
      if (tid == 0 && slice0 == 0) flag(p.status, 1u);
      const uint32_t cols = nslices * WAVES * NBW * 16;
      for (uint32_t i = tid; i < rows * cols; i += WAVES * 64) {
        const uint32_t r = i / cols;
        const uint32_t col = slice0 * WAVES * NBW * 16 + i % cols;
        if (col < N) ActBF16::store(p.out, static_cast<size_t>(row0 + r) * N + col, 0.0f);
      }
      return;
    }
  }
  const uint32_t mbu = (rows + 15) / 16;  // block-uniform, 1..kMB
  if constexpr (kMB >= 6) {
    if (mbu >= 6) return grouped_tile<EPI, WAVES, NBW, PROJ, TAIL, 6, WNT, TR>(p, w, row0, rows, slice0, nslices, s_a0);
  }
  if constexpr (kMB >= 5) {
    if (mbu >= 5) return grouped_tile<EPI, WAVES, NBW, PROJ, TAIL, 5, WNT, TR>(p, w, row0, rows, slice0, nslices, s_a0);
  }
  if constexpr (kMB >= 4) {
    if (mbu >= 4) return grouped_tile<EPI, WAVES, NBW, PROJ, TAIL, 4, WNT, TR>(p, w, row0, rows, slice0, nslices, s_a0);
  }
  if constexpr (kMB >= 3) {
    if (mbu >= 3) return grouped_tile<EPI, WAVES, NBW, PROJ, TAIL, 3, WNT, TR>(p, w, row0, rows, slice0, nslices, s_a0);
  }
  if constexpr (kMB >= 2) {
    if (mbu >= 2) return grouped_tile<EPI, WAVES, NBW, PROJ, TAIL, 2, WNT, TR>(p, w, row0, rows, slice0, nslices, s_a0);
  }
  grouped_tile<EPI, WAVES, NBW, PROJ, TAIL, 1, WNT, TR>(p, w, row0, rows, slice0, nslices, s_a0);
}

// ------------------------------------------------------------- row tiles ---

// Small calls: every tile holds at most 16 rows of one group (one MFMA row
// block), so the chunked GEMM's per-chunk A staging and barriers would only
// serialise the weight stream.  Here the block stages its tile's A rows over
// the whole K in LDS once and each wave streams its own 16 weight columns of
// every projection straight into its MFMA lanes, kRowsDepth chunks ahead,
// with no barrier in the K loop.
//
// K order: lane quarter q = lane / 16 owns the contiguous quarter of the
// groups [q G/4, (q + 1) G/4); MFMA step j feeds packed word j % 4 of the
// quarter's group j / 4.  So a lane's scales and biases for the whole K are
// 2 KCH contiguous bf16 values (loaded once per tile with wide loads: 2-byte
// loads per lane and chunk had cost more than the weights), and its weights
// of a chunk (two groups) are 32 contiguous bytes.  The fp32 sums over K run
// in a different order from the chunked GEMM, within the same tolerance.
// A row r stores its 16-byte unit u at (u & ~15) | ((u ^ rows_swz(r, q)) & 15):
// at step j the 64 lanes (16 rows x 4 quarters) read units q G/4*4 + j, which
// this spreads over all 16 bank groups, four lanes each.
constexpr int kRowsDepth = 3;  // chunks of weight loads in flight per wave
constexpr int kRowsCG = 8;     // 32-input groups per k_rows chunk (K = 256 KCH)

__device__ __forceinline__ constexpr uint32_t rows_swz(uint32_t r, uint32_t q) { return (r ^ (q << 2)) & 15u; }

// n consecutive dwords from a 4-byte aligned address, in the widest loads
template <int N>
__device__ __forceinline__ void ldg_dwords(const uint8_t* src, uint32_t (&out)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const uint4 v = ldg16(src + 4 * i);
      out[i] = v.x; out[i + 1] = v.y; out[i + 2] = v.z; out[i + 3] = v.w;
    }
  } else if constexpr (N == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(src);
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = *reinterpret_cast<const uint32_t*>(src + 4 * i);
  }
}

// One (tile, column slice) item of block-uniform index `item`; false when the
// item is past the live tiles.  KCH: K = 256 KCH (the instance is picked per
// K), so the kernel is straight-line and every wait counts exactly the loads
// it needs.  Load order: the tile's row indices (lanes 0-15), its A rows, the
// lane's scales and biases, the first kRowsDepth chunks of weights; the A
// rows go to LDS as they arrive, with the weight loads still in flight.
template <int EPI, int WAVES, int PROJ, int KCH>
__device__ __forceinline__ bool rows_item(const GroupedLaunch& p, uint32_t item, uint8_t* s_a, PhaseTrace& tr) {
  constexpr int kThreads = WAVES * 64;
  constexpr int kCols = WAVES * 16;
  constexpr int kG = KCH * kRowsCG;                // groups of K
  constexpr int kQG = kG / 4;                      // groups per lane quarter (2 KCH)
  constexpr int kUnits = kG * 4;                   // 16-byte A units per row
  constexpr int kRowBytes = kUnits * 16;
  static_assert((16 * kUnits) % kThreads == 0, "whole A units per thread");
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t K = p.k_dim, N = p.n_dim;

  // XCD-aware order: the column slices of a tile take consecutive blocks of
  // one XCD (block L runs on XCD L % 8) and share its L2 copy of the A rows
  const uint32_t slices = (N + kCols - 1) / kCols;
  const uint32_t r8 = item >> 3;
  const uint32_t slice = r8 % slices;
  const uint32_t tile = (r8 / slices) * 8 + (item & 7u);
  if (tile >= *p.tile_count) return false;
  const uint2 td = p.tiles[tile];
  const uint32_t group = td.x;
  const uint32_t row0 = p.row_off[group] + td.y;
  const uint32_t rows = min(p.row_off[group + 1] - row0, 16u);

  // the A row of each of the tile's rows, held by lanes 0-15 of every wave
  uint32_t my_row = row0;
  if (lane < rows) my_row = p.row_token != nullptr ? p.row_token[row0 + lane] : row0 + lane;

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
    if (tid == 0 && slice == 0) flag(p.status, 1u);
    for (uint32_t i = tid; i < rows * kCols; i += kThreads) {
      const uint32_t col = slice * kCols + i % kCols;
      if (col < N) ActBF16::store(p.out, static_cast<size_t>(row0 + i / kCols) * N + col, 0.0f);
    }
    return true;
  }
  if (p.trace != nullptr) tr.mark(1);

  // B: lane -> column lane % 16 of the wave's block, quarter q = lane / 16;
  // columns past N read the last row and are not stored
  const uint32_t bn = lane & 15u, q = lane >> 4;
  const uint32_t n_col = slice * kCols + wave * 16 + bn;
  const uint32_t col_ld = min(n_col, N - 1);
  const uint32_t g_lane = q * kQG;                 // the lane's first group
  uint32_t sv[PROJ][KCH], bv[PROJ][KCH];           // bf16 pairs of groups g_lane + 2 i, + 2 i + 1
  const uint8_t* wl[PROJ];
#pragma unroll
  for (int pj = 0; pj < PROJ; ++pj)
    wl[pj] = reinterpret_cast<const uint8_t*>(w[pj].w) + (static_cast<size_t>(col_ld) * kG + g_lane) * 16u;
  constexpr int kDepth = KCH < kRowsDepth ? KCH : kRowsDepth;
  uint4 bw[kDepth][PROJ][2];
  // the lane's scales and biases, then the first kDepth chunks of weights
  auto b_issue = [&]() {
#pragma unroll
    for (int pj = 0; pj < PROJ; ++pj) {
      const size_t m = (static_cast<size_t>(col_ld) * kG + g_lane) * 2u;
      ldg_dwords<KCH>(reinterpret_cast<const uint8_t*>(w[pj].s) + m, sv[pj]);
      ldg_dwords<KCH>(reinterpret_cast<const uint8_t*>(w[pj].b) + m, bv[pj]);
    }
    // keep the prefetch here and in chunk order: the scheduler otherwise sinks
    // every chunk's loads to just before their first use, or mixes the chunks,
    // and each chunk then waits for all outstanding loads
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
#pragma unroll
      for (int pj = 0; pj < PROJ; ++pj) {
        bw[d][pj][0] = ldg16(wl[pj] + d * 32u);
        bw[d][pj][1] = ldg16(wl[pj] + d * 32u + 16u);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // A rows: R rows of the tile are loaded (R = 4, 8 or 16, the least that
  // holds it and gives every thread whole units); LDS rows past R keep stale
  // data, which only reaches MFMA output rows that are not stored (an output
  // row depends on its own A row only).  Unit it = j * threads + tid -> (row
  // it / kUnits, unit it % kUnits).  The loads are unconditional (branches
  // here made every load wait for the one before): rows past the tile reload
  // its last row.
  const bool gather = p.row_token != nullptr;
  auto stage = [&](auto rows_class) {
    constexpr int R = decltype(rows_class)::value;
    constexpr int kIt = R * kUnits / kThreads;
    uint4 av[kIt];
#pragma unroll
    for (int j = 0; j < kIt; ++j) {
      const uint32_t it = j * kThreads + tid;
      const uint32_t r = min(it / kUnits, rows - 1), u = it % kUnits;
      uint32_t arow;
      if constexpr (kUnits % 64 == 0) {  // r is wave-uniform
        arow = gather ? __builtin_amdgcn_readlane(my_row, __builtin_amdgcn_readfirstlane(r)) : row0 + r;
      } else {
        arow = gather ? __shfl(my_row, static_cast<int>(r), 64) : row0 + r;
      }
      av[j] = ldg16(p.a + static_cast<size_t>(arow) * p.a_stride + u * 8u);
    }
    b_issue();
    if (p.trace != nullptr) tr.mark(2);
#pragma unroll
    for (int j = 0; j < kIt; ++j) {
      const uint32_t it = j * kThreads + tid;
      const uint32_t r = it / kUnits, u = it % kUnits;
      const uint4 x = av[j];
      const uint4 pp = kNatural ? x
                                : make_uint4((x.x & 0xffffu) | (x.z << 16), (x.x >> 16) | (x.z & 0xffff0000u),
                                             (x.y & 0xffffu) | (x.w << 16), (x.y >> 16) | (x.w & 0xffff0000u));
      const uint32_t phys = (u & ~15u) | ((u ^ rows_swz(r, u / (kQG * 4))) & 15u);
      *reinterpret_cast<uint4*>(s_a + r * kRowBytes + phys * 16u) = pp;
    }
  };
  constexpr bool kR4 = (4 * kUnits) % kThreads == 0, kR8 = (8 * kUnits) % kThreads == 0;
  if (kR4 && rows <= 4) stage(std::integral_constant<int, kR4 ? 4 : 16>{});
  else if (kR8 && rows <= 8) stage(std::integral_constant<int, kR8 ? 8 : 16>{});
  else stage(std::integral_constant<int, 16>{});
  __syncthreads();
  if (p.trace != nullptr) tr.mark(3);

  f32x4_t acc[PROJ];
#pragma unroll
  for (int pj = 0; pj < PROJ; ++pj) acc[pj] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t magic = f16_magic();
  const uint32_t am = lane & 15u;
  const uint8_t* a_lane = s_a + am * kRowBytes;
  const uint32_t a_sw = rows_swz(am, q);
  const uint32_t u_lane = q * kQG * 4;             // the lane's first A unit
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    const int d = c % kDepth;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int gi = 2 * c + (st >> 2);            // group of the lane's quarter
      const uint32_t u = u_lane + gi * 4 + (st & 3);
      const uint32_t phys = (u & ~15u) | ((u ^ a_sw) & 15u);
      const bf16x8_t aop = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(a_lane + phys * 16u));
#pragma unroll
      for (int pj = 0; pj < PROJ; ++pj) {
        const uint32_t s2 = sv[pj][gi >> 1], b2 = bv[pj][gi >> 1];
        const Dequant dq(__uint_as_float((gi & 1) ? s2 & 0xffff0000u : s2 << 16),
                         __uint_as_float((gi & 1) ? b2 & 0xffff0000u : b2 << 16));
        const uint4 wv = bw[d][pj][st >> 2];
        const int i = st & 3;
        uint32_t r4[4];
        dq.word(i == 0 ? wv.x : i == 1 ? wv.y : i == 2 ? wv.z : wv.w, magic, r4);
        acc[pj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, as_operand(r4), acc[pj], 0, 0, 0);
      }
    }
    if (c + kDepth < KCH) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int pj = 0; pj < PROJ; ++pj) {
        bw[d][pj][0] = ldg16(wl[pj] + (c + kDepth) * 32u);
        bw[d][pj][1] = ldg16(wl[pj] + (c + kDepth) * 32u + 16u);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if (p.trace != nullptr) tr.mark(4);
  // epilogue: lane holds rows 4 (lane / 16) + i, column lane % 16
  if (n_col >= N) return true;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t r = 4 * q + i;
    if (r >= rows) continue;
    const size_t o = static_cast<size_t>(row0 + r) * N + n_col;
    if constexpr (EPI == kEpiSwiglu) {
      ActBF16::store(p.out, o, swiglu_act<ActBF16>(round_bf16(acc[0][i]), round_bf16(acc[PROJ - 1][i])));
    } else {
      ActBF16::store(p.out, o, round_bf16(acc[0][i]));
    }
  }
  return true;
}

// One item per block over the bound of the live tiles (blocks past them exit).
// A loop of items per block kept loop-invariant arguments live and took the
// registers of a second block per CU.
template <int EPI, int WAVES, int PROJ, int KCH>
__global__ __launch_bounds__(WAVES * 64) void k_rows(GroupedLaunch p) {
  static_assert(EPI == kEpiSwiglu || EPI == kEpiRows, "Q4 epilogues only");
  extern __shared__ uint4 s_dyn[];
  uint8_t* s_a = reinterpret_cast<uint8_t*>(s_dyn);
  PhaseTrace tr;
  if (p.trace != nullptr) tr.mark(0);
  const bool live = rows_item<EPI, WAVES, PROJ, KCH>(p, blockIdx.x, s_a, tr);
  if (p.trace != nullptr && threadIdx.x == 0) {
    tr.mark(5);
    tr.t[7] = live ? 1u : 0u;
    tr.write(p.trace, EPI == kEpiSwiglu ? 7 : 8, blockIdx.x);
  }
}

// ------------------------------------------------------------------ sort ---

// Inclusive scan of one value per thread over a block of 1024 threads.
__device__ uint32_t block_scan_1024(uint32_t v, uint32_t* s_wave) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t u = __shfl_up(v, d, 64);
    if (lane >= static_cast<uint32_t>(d)) v += u;
  }
  if (lane == 63) s_wave[wave] = v;
  __syncthreads();
  uint32_t before = 0;
  for (uint32_t i = 0; i < wave; ++i) before += s_wave[i];
  __syncthreads();
  return v + before;
}

// Row offsets, both tile lists (group, first row) of the gate/up and the down
// tiles, from the row count n of group g = threadIdx.x (one block of 1024
// threads).  Returns the group's first row.
__device__ uint32_t sort_layout(const SortLaunch& p, uint32_t n, uint32_t* s_wave, bool write = true) {
  const uint32_t g = threadIdx.x;
  const uint32_t groups = p.experts + (p.shared_rows != 0 ? 1u : 0u);
  const uint32_t nt = (n + p.tile_rows - 1) / p.tile_rows;
  const uint32_t nt_dn = (n + p.tile_rows_dn - 1) / p.tile_rows_dn;
  const uint32_t row_end = block_scan_1024(n, s_wave);
  const uint32_t tile_end = block_scan_1024(nt, s_wave);
  const uint32_t tile_end_dn = block_scan_1024(nt_dn, s_wave);
  const uint32_t row_begin = row_end - n, tile_begin = tile_end - nt, tile_begin_dn = tile_end_dn - nt_dn;
  if (!write) return row_begin;
  if (g < groups) {
    p.row_off[g] = row_begin;
    for (uint32_t i = 0; i < nt; ++i) p.tiles[tile_begin + i] = make_uint2(g, i * p.tile_rows);
    for (uint32_t i = 0; i < nt_dn; ++i) p.tiles_dn[tile_begin_dn + i] = make_uint2(g, i * p.tile_rows_dn);
  }
  if (g == groups - 1) {
    p.row_off[groups] = row_end;
    *p.tile_count = tile_end;
    *p.tile_count_dn = tile_end_dn;
  }
  return row_begin;
}

// The whole sort in one block (small calls): LDS histogram of the routes, the
// layout (sort_layout), LDS cursors, scatter.  groups = experts (+1 for the
// shared rows) <= 1024.
__global__ __launch_bounds__(1024) void k_sort(SortLaunch p) {
  __shared__ uint32_t s_count[1024];
  __shared__ uint32_t s_wave[16];
  __shared__ uint32_t s_shared_first;
  const uint32_t g = threadIdx.x;
  const uint32_t pairs = p.tokens * p.slots;
  const uint32_t groups = p.experts + (p.shared_rows != 0 ? 1u : 0u);
  s_count[g] = 0;
  __syncthreads();
  for (uint32_t i = g; i < pairs; i += 1024) {
    const uint32_t e = static_cast<uint32_t>(p.inds[i]);
    if (e < p.experts) atomicAdd(&s_count[e], 1u);
    else flag(p.status, 2u);
  }
  __syncthreads();
  uint32_t n = 0;
  if (g < p.experts) n = s_count[g];
  else if (g < groups) n = p.shared_rows;
  const uint32_t row_begin = sort_layout(p, n, s_wave);
  if (g == p.experts) s_shared_first = row_begin;
  s_count[g] = row_begin;  // scatter cursors
  __syncthreads();
  for (uint32_t i = g; i < pairs; i += 1024) {
    const uint32_t e = static_cast<uint32_t>(p.inds[i]);
    if (e < p.experts) {
      const uint32_t pos = atomicAdd(&s_count[e], 1u);
      p.row_token[pos] = i / p.slots;
      p.pair_row[i] = pos;
    } else {
      p.pair_row[i] = kNoRow;
    }
  }
  for (uint32_t i = g; i < p.shared_rows; i += 1024) p.row_token[s_shared_first + i] = i;
}

// The sort of large calls over many blocks (the scattered row writes of one
// block were the cost): zero the counts, per-block LDS histograms added to
// global counts, one block lays out rows and tiles, then every block reserves
// each expert's run of rows with one atomic and scatters its pairs into it.
// The order of an expert's rows then depends on which block reserved first,
// which changes no result: every output row is its own set of dot products.
constexpr int kSortThreads = 256;
constexpr int kSortPerThread = 8;
constexpr uint32_t kSortBlockPairs = kSortThreads * kSortPerThread;

__global__ __launch_bounds__(1024) void k_sort_zero(SortLaunch p) { p.counts[threadIdx.x] = 0; }

__global__ __launch_bounds__(kSortThreads) void k_sort_count(SortLaunch p) {
  __shared__ uint32_t s_count[1024];
  const uint32_t tid = threadIdx.x;
  const uint32_t pairs = p.tokens * p.slots;
  const uint32_t base = blockIdx.x * kSortBlockPairs;
  for (uint32_t g = tid; g < 1024; g += kSortThreads) s_count[g] = 0;
  __syncthreads();
  uint32_t e[kSortPerThread];
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j)
    e[j] = static_cast<uint32_t>(p.inds[min(base + j * kSortThreads + tid, pairs - 1)]);
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j) {
    if (base + j * kSortThreads + tid >= pairs) continue;
    if (e[j] < p.experts) atomicAdd(&s_count[e[j]], 1u);
    else flag(p.status, 2u);
  }
  __syncthreads();
  for (uint32_t g = tid; g < p.experts; g += kSortThreads)
    if (s_count[g] != 0) atomicAdd(&p.counts[g], s_count[g]);
}

__global__ __launch_bounds__(1024) void k_sort_scan(SortLaunch p) {
  __shared__ uint32_t s_wave[16];
  __shared__ uint32_t s_shared_first;
  const uint32_t g = threadIdx.x;
  const uint32_t groups = p.experts + (p.shared_rows != 0 ? 1u : 0u);
  uint32_t n = 0;
  if (g < p.experts) n = p.counts[g];
  else if (g < groups) n = p.shared_rows;
  const uint32_t row_begin = sort_layout(p, n, s_wave);
  if (g == p.experts) s_shared_first = row_begin;
  p.cursors[g] = row_begin;
  __syncthreads();
  for (uint32_t i = g; i < p.shared_rows; i += 1024) p.row_token[s_shared_first + i] = i;
}

__global__ __launch_bounds__(kSortThreads) void k_sort_scatter(SortLaunch p) {
  __shared__ uint32_t s_count[1024];
  __shared__ uint32_t s_base[1024];
  const uint32_t tid = threadIdx.x;
  const uint32_t pairs = p.tokens * p.slots;
  const uint32_t base = blockIdx.x * kSortBlockPairs;
  for (uint32_t g = tid; g < 1024; g += kSortThreads) s_count[g] = 0;
  __syncthreads();
  uint32_t e[kSortPerThread], local[kSortPerThread];
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j)
    e[j] = static_cast<uint32_t>(p.inds[min(base + j * kSortThreads + tid, pairs - 1)]);
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j) {
    local[j] = 0;
    if (base + j * kSortThreads + tid < pairs && e[j] < p.experts) local[j] = atomicAdd(&s_count[e[j]], 1u);
  }
  __syncthreads();
  for (uint32_t g = tid; g < p.experts; g += kSortThreads)
    if (s_count[g] != 0) s_base[g] = atomicAdd(&p.cursors[g], s_count[g]);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kSortPerThread; ++j) {
    const uint32_t i = base + j * kSortThreads + tid;
    if (i >= pairs) continue;
    if (e[j] < p.experts) {
      const uint32_t pos = s_base[e[j]] + local[j];
      p.row_token[pos] = i / p.slots;
      p.pair_row[i] = pos;
    } else {
      p.pair_row[i] = kNoRow;
    }
  }
}

// The layout and scatter of the sort when k_sort_count has filled p.counts
// and p.cursors was zeroed before it: one launch.  Every block lays the rows
// out from the counts (the same scans; block 0 writes the row offsets, tile
// lists and the shared rows' tokens), counts its own pairs in LDS, reserves
// each expert's run of rows with one atomic on the zeroed cursor and scatters
// its pairs into it.
constexpr uint32_t kPlacePerThread = 2;
constexpr uint32_t kPlaceBlockPairs = 1024 * kPlacePerThread;

__global__ __launch_bounds__(1024) void k_sort_place(SortLaunch p) {
  __shared__ uint32_t s_wave[16];
  __shared__ uint32_t s_count[1024];
  __shared__ uint32_t s_base[1024];
  __shared__ uint32_t s_shared_first;
  const uint32_t g = threadIdx.x;
  const uint32_t pairs = p.tokens * p.slots;
  const uint32_t groups = p.experts + (p.shared_rows != 0 ? 1u : 0u);
  const uint32_t base = blockIdx.x * kPlaceBlockPairs;
  uint32_t e[kPlacePerThread];
#pragma unroll
  for (uint32_t j = 0; j < kPlacePerThread; ++j)
    e[j] = static_cast<uint32_t>(p.inds[min(base + j * 1024 + g, pairs - 1)]);
  uint32_t n = 0;
  if (g < p.experts) n = p.counts[g];
  else if (g < groups) n = p.shared_rows;
  s_count[g] = 0;
  const uint32_t row_begin = sort_layout(p, n, s_wave, blockIdx.x == 0);
  if (g == p.experts) s_shared_first = row_begin;
  uint32_t local[kPlacePerThread];
#pragma unroll
  for (uint32_t j = 0; j < kPlacePerThread; ++j) {
    local[j] = 0;
    if (base + j * 1024 + g < pairs && e[j] < p.experts) local[j] = atomicAdd(&s_count[e[j]], 1u);
  }
  __syncthreads();
  if (g < p.experts && s_count[g] != 0) s_base[g] = row_begin + atomicAdd(&p.cursors[g], s_count[g]);
  __syncthreads();
#pragma unroll
  for (uint32_t j = 0; j < kPlacePerThread; ++j) {
    const uint32_t i = base + j * 1024 + g;
    if (i >= pairs) continue;
    if (e[j] < p.experts) {
      const uint32_t pos = s_base[e[j]] + local[j];
      p.row_token[pos] = i / p.slots;
      p.pair_row[i] = pos;
    } else {
      p.pair_row[i] = kNoRow;
      flag(p.status, 2u);
    }
  }
  if (blockIdx.x == 0)
    for (uint32_t i = g; i < p.shared_rows; i += 1024) p.row_token[s_shared_first + i] = i;
}

// --------------------------------------------------------------- combine ---

// A token's value of a [tokens, ...] array.  UNIFORM: the address is the same
// in every lane of the wave, and the value is read through the scalar data
// cache into SGPRs (the arrays read this way are written by earlier
// launches only).
template <bool UNIFORM>
__device__ __forceinline__ uint32_t token_u32(const uint32_t* p, size_t i) {
  if constexpr (UNIFORM) return *(const __attribute__((address_space(4))) uint32_t*)(p + i);
  else return p[i];
}
// Element i of a bf16 (dtype 0) or fp32 array in two steps, so that a scalar
// load's wait comes at the value's first use rather than at the load: the
// raw dword (UNIFORM: the aligned dword holding a bf16 element, which never
// crosses a page) and its conversion.
struct TokenRaw {
  uint32_t w, high;
};
template <bool UNIFORM>
__device__ __forceinline__ TokenRaw token_raw(const void* p, size_t i, uint32_t dtype) {
  if constexpr (UNIFORM) {
    if (dtype != 0) return {token_u32<true>(static_cast<const uint32_t*>(p), i), 2u};
    const uintptr_t a = reinterpret_cast<uintptr_t>(p) + 2u * i;
    return {*(const __attribute__((address_space(4))) uint32_t*)(a & ~static_cast<uintptr_t>(3)),
            static_cast<uint32_t>(a & 2u) >> 1};
  } else {
    return {dtype != 0 ? ldg_u32(static_cast<const float*>(p) + i) : ldg_u16(static_cast<const uint16_t*>(p) + i),
            dtype != 0 ? 2u : 0u};
  }
}
// high: 0 low bf16 half, 1 high bf16 half, 2 fp32
__device__ __forceinline__ float token_value(TokenRaw r) {
  return r.high == 2u ? __uint_as_float(r.w) : bf16_to_f32(r.high ? r.w >> 16 : r.w & 0xffffu);
}
template <bool UNIFORM>
__device__ __forceinline__ float token_any(const void* p, size_t i, uint32_t dtype) {
  return token_value(token_raw<UNIFORM>(p, i, dtype));
}

// One thread per 8 outputs of one token.  mode 1 (generic): products rounded,
// summed in slot order in fp32, rounded; mode 0 (fused): fp32 sum of
// round(down) * score.  Then + round(sigmoid gate * shared) or + shared_y.
// mode 2: no combine, out[t, j] = the slot's expert output row.
// WAVE_TOKEN (hidden / 8 a multiple of 64): the 64 threads of a wave hold
// outputs of one token, so its row indices, scores and gates are scalar
// loads and each row load is an SGPR base plus the lane's offset; the
// registers that frees let every wave of a 2048-token call be resident at
// once (at most 64 VGPRs: eight waves per SIMD).
template <bool WAVE_TOKEN>
__global__ __launch_bounds__(kGB) void k_grouped_combine(CombineLaunch p) {
  const uint32_t per_token = p.hidden / 8;
  const uint32_t i = blockIdx.x * kGB + threadIdx.x;
  if (i >= p.tokens * per_token) return;
  uint32_t t = i / per_token;
  if constexpr (WAVE_TOKEN) t = __builtin_amdgcn_readfirstlane(t);
  const uint32_t h0 = (i % per_token) * 8;
  // the pointers the first loads need, read from the arguments together, so
  // that the token's index loads and the shared row's are issued together
  const uint32_t* pair_row = p.pair_row;
  const uint32_t* shared_first = p.shared_first;
  VM_KEEP(pair_row);
  VM_KEEP(shared_first);
  const uint32_t voff = h0 * 2u;  // the lane's byte offset in a row
  auto row_ptr = [&](uint32_t row) {
    return reinterpret_cast<const uint8_t*>(p.rows + static_cast<size_t>(row) * p.hidden) + voff;
  };
  if (p.mode == 2) {  // no combine: every slot's rounded expert output
    for (uint32_t j = 0; j < p.slots; ++j) {
      const uint32_t row = token_u32<WAVE_TOKEN>(pair_row, static_cast<size_t>(t) * p.slots + j);
      const uint4 v = row == kNoRow ? make_uint4(0, 0, 0, 0) : ldg16(row_ptr(row));
      *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + (static_cast<size_t>(t) * p.slots + j) * p.hidden +
                                h0) = v;
    }
    return;
  }
  // every load of the token is issued before the sums (slots <= kCombineSlots):
  // row indices and scores, then the expert rows and the shared row, so the
  // thread waits for one round trip of each kind rather than one per slot
  uint32_t row[kCombineSlots];
  float sc[kCombineSlots];
  const uint32_t first = shared_first != nullptr ? token_u32<WAVE_TOKEN>(shared_first, 0) : 0u;
#pragma unroll
  for (int j = 0; j < kCombineSlots; ++j)
    row[j] = j < static_cast<int>(p.slots) ? token_u32<WAVE_TOKEN>(pair_row, static_cast<size_t>(t) * p.slots + j)
                                           : kNoRow;
  uint4 sh = make_uint4(0, 0, 0, 0);
  TokenRaw sig_raw{0u, 2u};
  const uint16_t* shr = shared_first != nullptr ? p.rows + static_cast<size_t>(first) * p.hidden : p.shared_rows;
  if (shr != nullptr) {
    sh = ldg16(reinterpret_cast<const uint8_t*>(shr + static_cast<size_t>(t) * p.hidden) + voff);
    sig_raw = token_raw<WAVE_TOKEN>(p.shared_sig, t, 0);
  } else if (p.shared_y != nullptr) {
    sh = ldg16(reinterpret_cast<const uint8_t*>(static_cast<const uint16_t*>(p.shared_y) +
                                                static_cast<size_t>(t) * p.hidden) + voff);
  }
  uint4 v[kCombineSlots];
#pragma unroll
  for (int j = 0; j < kCombineSlots; ++j) v[j] = row[j] != kNoRow ? ldg16(row_ptr(row[j])) : make_uint4(0, 0, 0, 0);
  TokenRaw sr[kCombineSlots];
#pragma unroll
  for (int j = 0; j < kCombineSlots; ++j)
    sr[j] = row[j] != kNoRow ? token_raw<WAVE_TOKEN>(p.scores, static_cast<size_t>(t) * p.slots + j, p.score_dtype)
                             : TokenRaw{0u, 2u};
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < kCombineSlots; ++j) {
    if (row[j] == kNoRow) continue;
    sc[j] = token_value(sr[j]);
    const uint32_t words[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = bf16_to_f32(e & 1 ? words[e / 2] >> 16 : words[e / 2] & 0xffffu);
      const float prod = __fmul_rn(d, sc[j]);
      acc[e] = __fadd_rn(acc[e], p.mode == 1 ? round_bf16(prod) : prod);
    }
  }
  const float sig = token_value(sig_raw);
  uint32_t out[4];
  const uint32_t shw[4] = {sh.x, sh.y, sh.z, sh.w};
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float y[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float v = round_bf16(acc[e + k]);
      const float s = bf16_to_f32(k ? shw[e / 2] >> 16 : shw[e / 2] & 0xffffu);
      if (shr != nullptr) v = round_bf16(__fadd_rn(v, round_bf16(__fmul_rn(sig, s))));
      else if (p.shared_y != nullptr) v = round_bf16(__fadd_rn(v, s));
      y[k] = v;
    }
    out[e / 2] = f32_to_bf16(y[0]) | (f32_to_bf16(y[1]) << 16);
  }
  *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + static_cast<size_t>(t) * p.hidden + h0) =
      make_uint4(out[0], out[1], out[2], out[3]);
  // the hyper-connection injection of the 8 combined values into every stream
  const Inject& inj = p.inject;
  if (inj.out == nullptr) return;
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = bf16_to_f32(e & 1 ? out[e / 2] >> 16 : out[e / 2] & 0xffffu);
  for (uint32_t j = 0; j < inj.hc; ++j) {
    const size_t o = (static_cast<size_t>(t) * inj.hc + j) * p.hidden + h0;
    const float w = token_any<WAVE_TOKEN>(inj.weights, static_cast<size_t>(t) * inj.hc + j, 0);
    const uint4 hv = ldg16(static_cast<const uint16_t*>(inj.hidden) + o);
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
    uint32_t res[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float v[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const float h = bf16_to_f32(k ? hw[e / 2] >> 16 : hw[e / 2] & 0xffffu);
        v[k] = round_bf16(__fadd_rn(h, round_bf16(__fmul_rn(y[e + k], w))));
      }
      res[e / 2] = f32_to_bf16(v[0]) | (f32_to_bf16(v[1]) << 16);
    }
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(inj.out) + o) = make_uint4(res[0], res[1], res[2], res[3]);
  }
}

// ----------------------------------------------------------- shared gate ---

// sigmoid(round(x . dequant(seg))) per token, one wave per token (bf16).
__global__ __launch_bounds__(64) void k_shared_gate(const uint16_t* x, ProjPtrs seg, uint16_t* sig, uint32_t hidden) {
  const uint32_t t = blockIdx.x, lane = threadIdx.x;
  const float logit = shared_gate_logit_bf16(x + static_cast<size_t>(t) * hidden, seg, hidden, lane);
  if (lane == 0) ActBF16::store(sig, t, sigmoid_act<ActBF16>(logit));
}

// ------------------------------------------------------------ dispatch ----

template <class... KArgs, class... Args>
hipError_t launch(const char* family, void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream,
                  Args... args) {
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events(family, &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
  return hipGetLastError();
}

template <int EPI, int WAVES, int NBW, int PROJ, bool TAIL, bool WNT, int TR = tile_rows<EPI>()>
hipError_t grouped_go_k(const char* family, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  // one LDS stage with staged weights (see grouped_tile), else two
  constexpr uint32_t lds = (lds_weights<EPI, TAIL>() ? 1 : 2) * stage_bytes<EPI, WAVES, NBW, PROJ, TAIL, TR>();
  static_assert(lds <= 160u * 1024u, "the LDS of one block");
  auto kernel = &k_grouped<EPI, WAVES, NBW, PROJ, TAIL, WNT, TR>;
  static bool attr = false;  // one attribute call per kernel instance
  if (!attr) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr = true;
  }
  const uint32_t cols = WAVES * NBW * 16;
  const uint32_t slices = (p.n_dim + cols - 1) / cols;
  // slices per block: the one-stage path only, and a divisor of the slices
  uint32_t spb = lds_weights<EPI, TAIL>() && p.n_dim % cols == 0 ? slices_per_block<EPI>() : 1u;
  while (slices % spb != 0) spb /= 2;
  GroupedLaunch q = p;
  q.spb = spb;
  const dim3 grid(slices / spb * ((max_tiles + 7) / 8 * 8));
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events(family, &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, dim3(WAVES * 64), lds, stream, start, stop, 0, q);
  else
    hipLaunchKernelGGL(kernel, grid, dim3(WAVES * 64), lds, stream, q);
  return hipGetLastError();
}

template <int EPI, int WAVES, int NBW, int PROJ>
hipError_t grouped_go(const char* family, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  if constexpr (EPI == kEpiSwiglu || EPI == kEpiRows) {
    // tall tiles: calls of many rows per group, whose groups then need fewer
    // row tiles (each tile dequantises its expert's weights once); full
    // chunks and cached weight loads only
    if (p.tile_rows == static_cast<uint32_t>(kGroupedRowsTall)) {
      if ((p.k_dim / kGroup) % kCG != 0 || p.weights_once) return hipErrorInvalidValue;
      return grouped_go_k<EPI, WAVES, NBW, PROJ, false, false, kGroupedRowsTall>(family, p, max_tiles, stream);
    }
  }
  if (p.tile_rows != 0 && p.tile_rows != static_cast<uint32_t>(tile_rows<EPI>())) return hipErrorInvalidValue;
  if ((p.k_dim / kGroup) % kCG != 0)
    return grouped_go_k<EPI, WAVES, NBW, PROJ, true, false>(family, p, max_tiles, stream);
  if (lds_weights<EPI, false>() && p.weights_once)
    return grouped_go_k<EPI, WAVES, NBW, PROJ, false, lds_weights<EPI, false>()>(family, p, max_tiles, stream);
  return grouped_go_k<EPI, WAVES, NBW, PROJ, false, false>(family, p, max_tiles, stream);
}

}  // namespace

uint32_t grouped_max_tiles(uint32_t rows, uint32_t groups, uint32_t tile_rows) {
  return (rows + tile_rows - 1) / tile_rows + groups;
}

// block shapes (waves, 16-column blocks per wave) of the gate/up and down GEMMs
#ifndef VM_GU_WAVES
#define VM_GU_WAVES 4
#endif
#ifndef VM_GU_NBW
#define VM_GU_NBW 1
#endif
#ifndef VM_DN_WAVES
#define VM_DN_WAVES 8
#endif
#ifndef VM_DN_NBW
#define VM_DN_NBW 2
#endif

hipError_t launch_grouped(int epi, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  // the kernels address A, and each projection's weights, scales and biases,
  // with 32-bit byte offsets
  if (p.a_rows == 0 || static_cast<uint64_t>(p.a_rows) * p.a_stride * 2u > 0xffffffffull ||
      static_cast<uint64_t>(p.n_dim) * p.k_dim > 0xffffffffull)
    return hipErrorInvalidValue;
  // a call with no routed experts is the shared expert's own GEMM (run on a
  // side stream beside the routing), timed apart from the routed experts
  const bool own = p.experts == 0;
  switch (epi) {
    case kEpiSwiglu:
      return grouped_go<kEpiSwiglu, VM_GU_WAVES, VM_GU_NBW, 2>(own ? "shared_gateup" : "grouped_gateup", p,
                                                               max_tiles, stream);
    case kEpiRows:
      return grouped_go<kEpiRows, VM_DN_WAVES, VM_DN_NBW, 1>(own ? "shared_down" : "grouped_down", p, max_tiles,
                                                             stream);
    default: return grouped_go<kEpiLogits, 4, 1, 1>("router_gemm", p, max_tiles, stream);
  }
}

// The k_rows instances: K of 256, 512, 1024, 2048 or 4096 exactly (their
// strides are compile-time; the A rows of a 16-row tile take 8 to 128 KiB of
// LDS).  Other K take the chunked GEMM.
constexpr uint32_t kRowsMaxK = 4096;

bool rows_supported(uint32_t k_dim) {
  return k_dim == 256 || k_dim == 512 || k_dim == 1024 || k_dim == 2048 || k_dim == kRowsMaxK;
}

template <int EPI, int WAVES, int PROJ, int KCH>
hipError_t rows_go_k(const char* family, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  auto kernel = &k_rows<EPI, WAVES, PROJ, KCH>;
  constexpr uint32_t lds = 16u * KCH * kRowsCG * kGroup * 2u;
  static bool attr = false;  // one attribute call per kernel instance
  if (!attr) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr = true;
  }
  const uint32_t cols = WAVES * 16;
  const dim3 grid(((p.n_dim + cols - 1) / cols) * ((max_tiles + 7) / 8 * 8));
  GroupedLaunch q = p;
  q.trace = trace_reserve(grid.x);
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events(family, &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, dim3(WAVES * 64), lds, stream, start, stop, 0, q);
  else
    hipLaunchKernelGGL(kernel, grid, dim3(WAVES * 64), lds, stream, q);
  return hipGetLastError();
}

#ifndef VM_ROWS_GU_WAVES
#define VM_ROWS_GU_WAVES 4
#endif
#ifndef VM_ROWS_DN_WAVES
#define VM_ROWS_DN_WAVES 8
#endif

template <int EPI, int WAVES, int PROJ>
hipError_t rows_go(const char* family, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  switch (p.k_dim) {
    case 256: return rows_go_k<EPI, WAVES, PROJ, 1>(family, p, max_tiles, stream);
    case 512: return rows_go_k<EPI, WAVES, PROJ, 2>(family, p, max_tiles, stream);
    case 1024: return rows_go_k<EPI, WAVES, PROJ, 4>(family, p, max_tiles, stream);
    case 2048: return rows_go_k<EPI, WAVES, PROJ, 8>(family, p, max_tiles, stream);
    case 4096: return rows_go_k<EPI, WAVES, PROJ, 16>(family, p, max_tiles, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rows(int epi, const GroupedLaunch& p, uint32_t max_tiles, hipStream_t stream) {
  if (!rows_supported(p.k_dim)) return hipErrorInvalidValue;
  if (epi == kEpiSwiglu) return rows_go<kEpiSwiglu, VM_ROWS_GU_WAVES, 2>("grouped_gateup", p, max_tiles, stream);
  if (epi == kEpiRows) return rows_go<kEpiRows, VM_ROWS_DN_WAVES, 1>("grouped_down", p, max_tiles, stream);
  return hipErrorInvalidValue;
}


hipError_t launch_sort(const SortLaunch& p, hipStream_t stream) {
  const uint32_t pairs = p.tokens * p.slots;
  if (pairs <= kSortOneBlockPairs) return launch("sort", k_sort, dim3(1), dim3(1024), stream, p);
  const dim3 blocks((pairs + kSortBlockPairs - 1) / kSortBlockPairs);
  hipError_t e = launch("sort", k_sort_zero, dim3(1), dim3(1024), stream, p);
  if (e == hipSuccess) e = launch("sort", k_sort_count, blocks, dim3(kSortThreads), stream, p);
  if (e == hipSuccess) e = launch("sort", k_sort_scan, dim3(1), dim3(1024), stream, p);
  if (e == hipSuccess) e = launch("sort", k_sort_scatter, blocks, dim3(kSortThreads), stream, p);
  return e;
}

hipError_t launch_sort_counted(const SortLaunch& p, hipStream_t stream) {
  const uint32_t pairs = p.tokens * p.slots;
  hipError_t e = launch("sort", k_sort_count, dim3((pairs + kSortBlockPairs - 1) / kSortBlockPairs),
                        dim3(kSortThreads), stream, p);
  if (e == hipSuccess)
    e = launch("sort", k_sort_place, dim3((pairs + kPlaceBlockPairs - 1) / kPlaceBlockPairs), dim3(1024), stream, p);
  return e;
}

hipError_t launch_grouped_combine(const CombineLaunch& p, hipStream_t stream) {
  if (p.slots == 0 || p.slots > static_cast<uint32_t>(kCombineSlots)) return hipErrorInvalidValue;
  const uint32_t n = p.tokens * (p.hidden / 8);
  if ((p.hidden / 8) % 64 == 0)
    return launch("combine", k_grouped_combine<true>, dim3((n + kGB - 1) / kGB), dim3(kGB), stream, p);
  return launch("combine", k_grouped_combine<false>, dim3((n + kGB - 1) / kGB), dim3(kGB), stream, p);
}

hipError_t launch_shared_gate(const uint16_t* x, const ProjPtrs& seg, uint16_t* sig, uint32_t tokens,
                              uint32_t hidden, hipStream_t stream) {
  return launch("shared_gate", k_shared_gate, dim3(tokens), dim3(64), stream, x, seg, sig, hidden);
}

}  // namespace vm

// Device helpers shared by the gfx950 MoE kernels: activation types, bf16
// rounding, wave64 DPP reductions and the Q4/G32 group dot products.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vm {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kGroup = 32;            // Q4 affine group size (MLX G32)
constexpr int kWordsPerGroup = kGroup / 8;
constexpr uint32_t kSlotBit = 0x80000000u;

// ---------------------------------------------------------------- bf16 ----

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even float -> bf16 bits (gfx950 v_cvt_pk_bf16_f32); NaN
// stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Activation element types.  `round` is the rounding applied where the
// reference stores a value of the activation type.
struct ActBF16 {
  using T = uint16_t;
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ float round(float f) { return round_bf16(f); }
  __device__ static __forceinline__ float load(const void* p, size_t i) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static __forceinline__ void store(void* p, size_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16(v));
  }
  // raw element bits (the conversion, and so the wait, comes at from_bits)
  __device__ static __forceinline__ uint32_t load_bits(const void* p, size_t i);
  __device__ static __forceinline__ float from_bits(uint32_t b) { return bf16_to_f32(b); }
};

struct ActF32 {
  using T = float;
  static constexpr int kBytes = 4;
  __device__ static __forceinline__ float round(float f) { return f; }
  __device__ static __forceinline__ float load(const void* p, size_t i) {
    return static_cast<const float*>(p)[i];
  }
  __device__ static __forceinline__ void store(void* p, size_t i, float v) {
    static_cast<float*>(p)[i] = v;
  }
  __device__ static __forceinline__ uint32_t load_bits(const void* p, size_t i);
  __device__ static __forceinline__ float from_bits(uint32_t b) { return __uint_as_float(b); }
};

__device__ __forceinline__ float load_any(const void* p, size_t i, uint32_t dtype) {
  return dtype == 0 ? ActBF16::load(p, i) : ActF32::load(p, i);
}

// ------------------------------------------------------- global loads ---
// Loads through an explicit global-address-space pointer.  A pointer that
// went through readlane or a select is generic to the compiler, and generic
// (flat) loads also count on the LDS/scalar counter, so every LDS access or
// kernel-argument read after them waits for the whole stream.
typedef unsigned int vm_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ldg16(const void* p) {
  const vm_u32x4 v = *(const __attribute__((address_space(1))) vm_u32x4*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// A streaming load (non-temporal): data read once, kept from displacing
// reused lines in the L2.
__device__ __forceinline__ uint4 ldg16_nt(const void* p) {
  const vm_u32x4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) vm_u32x4*)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t ldg_u16(const void* p) {
  return *(const __attribute__((address_space(1))) unsigned short*)(p);
}

__device__ __forceinline__ uint32_t ldg_u32(const void* p) {
  return *(const __attribute__((address_space(1))) unsigned int*)(p);
}

__device__ __forceinline__ uint32_t ActBF16::load_bits(const void* p, size_t i) {
  return ldg_u16(static_cast<const uint16_t*>(p) + i);
}
__device__ __forceinline__ uint32_t ActF32::load_bits(const void* p, size_t i) {
  return ldg_u32(static_cast<const float*>(p) + i);
}

// Materialises a kernel-argument value in SGPRs at this point.  Members of a
// by-value kernel argument are otherwise read at their first use, which puts
// one scalar-load round trip per use on the critical path.
#define VM_PIN(value) asm volatile("" ::"s"(value))

// Keeps a uniform local copy of a kernel-argument value in SGPRs: after this
// the compiler cannot re-read it from the argument segment at a later use.
#define VM_KEEP(lvalue) asm volatile("" : "+s"(lvalue))

// ---------------------------------------------------------- activations --
// MLX's stable sigmoid sequence, every step rounded to the activation type
// (models/flashnext/metal_runtime.py:277-283), then silu(g) * u.

template <class A>
__device__ __forceinline__ float sigmoid_act(float g) {
#pragma clang fp contract(off)
  float mag = fabsf(g);
  float e = A::round(expf(mag));
  float den = A::round(1.0f + e);
  float small = A::round(1.0f / den);
  return g < 0.0f ? small : A::round(1.0f - small);
}

template <class A>
__device__ __forceinline__ float swiglu_act(float g, float u) {
#pragma clang fp contract(off)
  float s = A::round(g * sigmoid_act<A>(g));
  return A::round(s * u);
}

// Block barrier that orders LDS only: global stores stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------- reductions ---
// DPP controls (GFX9): quad_perm, row_half_mirror, row_mirror, row_bcast.
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7-i within 8
constexpr int kDppMirror = 0x140;      // lane i <- lane 15-i within 16
constexpr int kDppBcast15 = 0x142;     // row r <- lane 15 of row r-1
constexpr int kDppBcast31 = 0x143;     // rows 2,3 <- lane 31

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over aligned groups of N lanes (N = 1..64, power of two).  Afterwards
// lane (N-1) of every group (and for N <= 16 every lane) holds the group sum.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp_f<kDppQuadXor1>(v);
  if constexpr (N >= 4) v += dpp_f<kDppQuadXor2>(v);
  if constexpr (N >= 8) v += dpp_f<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp_f<kDppMirror>(v);
  if constexpr (N >= 32) v += dpp_f<kDppBcast15, 0xA>(v);
  if constexpr (N >= 64) v += dpp_f<kDppBcast31, 0xC>(v);
  return v;
}

// Wave-wide unsigned max, broadcast to every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u<kDppQuadXor1>(v));
  v = max(v, dpp_u<kDppQuadXor2>(v));
  v = max(v, dpp_u<kDppHalfMirror>(v));
  v = max(v, dpp_u<kDppMirror>(v));
  v = max(v, dpp_u<kDppBcast15, 0xA>(v));
  v = max(v, dpp_u<kDppBcast31, 0xC>(v));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, uint32_t lane) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), lane));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ float wave_sum_all(float v) {
  v = group_sum<64>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max_f32(float v) {
  // Works for any finite or infinite floats: max through DPP on floats.
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  // rows without a source keep their own value: use max with self via mask
  float t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      __builtin_bit_cast(int, v), __builtin_bit_cast(int, v), kDppBcast15, 0xA, 0xF, false));
  v = fmaxf(v, t);
  t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      __builtin_bit_cast(int, v), __builtin_bit_cast(int, v), kDppBcast31, 0xC, 0xF, false));
  v = fmaxf(v, t);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// ------------------------------------------------------- Q4 group dots ---
// One group = 32 consecutive inputs = 4 packed uint32 words; nibble n of word
// i is input 8*i + n (bits 4n..4n+3), the MLX order.
//
// bf16 activations: a nibble pair (n, n+4) of word i is turned into the bf16
// pair (128 + q_n, 128 + q_{n+4}) by one and/or with exponent 0x43 (=2^7), and
// multiplied with the activation pair (x_{8i+n}, x_{8i+n+4}) by v_dot2 with
// fp32 accumulation.  The dot then equals sum(q*x) + 128*sum(x); callers
// remove the 128*sum(x) term with the per-group activation sum.

// Repack 16 words of bf16 activations (natural pairs (x_2m, x_2m+1)) into the
// (x_{8i+n}, x_{8i+n+4}) pair order, index 4*i + n.
__device__ __forceinline__ void pair_activations(const uint32_t raw[16], uint32_t xp[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t a = raw[4 * i + 0], b = raw[4 * i + 1], c = raw[4 * i + 2], d = raw[4 * i + 3];
    xp[4 * i + 0] = (a & 0xffffu) | (c << 16);          // x0, x4
    xp[4 * i + 1] = (a >> 16) | (c & 0xffff0000u);      // x1, x5
    xp[4 * i + 2] = (b & 0xffffu) | (d << 16);          // x2, x6
    xp[4 * i + 3] = (b >> 16) | (d & 0xffff0000u);      // x3, x7
  }
}

__device__ __forceinline__ float bf16_pair_sum(const uint32_t raw[16]) {
  float s = 0.0f;
#pragma unroll
  for (int m = 0; m < 16; ++m) s += bf16_to_f32(raw[m] & 0xffffu) + bf16_to_f32(raw[m] >> 16);
  return s;
}

__device__ __forceinline__ float q4_dot_bf16(const uint4 w, const uint32_t xp[16]) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const uint32_t q = ((words[i] >> (4 * n)) & 0x000f000fu) | 0x43004300u;
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q),
                                           __builtin_bit_cast(bf16x2, xp[4 * i + n]), acc, false);
    }
  }
  return acc;
}

// fp32 activations: plain nibble extraction and FMA.
__device__ __forceinline__ float q4_dot_f32(const uint4 w, const float x[32]) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      acc = fmaf(static_cast<float>((words[i] >> (4 * n)) & 15u), x[8 * i + n], acc);
    }
  }
  return acc;
}

// ----------------------------------------------------- expert addressing --

struct ProjPtrs {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
};

// The shared expert's H -> 1 Q4 gate logit of one bf16 row, summed by one
// wave and rounded to bf16: the grouped path's shared gate kernel and the
// selection of calls that run the shared expert as a sorted group use this
// one sum.
__device__ __forceinline__ float shared_gate_logit_bf16(const uint16_t* x_row, const ProjPtrs& seg, uint32_t hidden,
                                                        uint32_t lane) {
  const uint32_t G = hidden / kGroup;
  float acc = 0.0f;
  for (uint32_t g = lane; g < G; g += 64) {
    const uint4 w = ldg16(seg.w + g * kWordsPerGroup);
    const uint16_t* src = x_row + g * kGroup;
    uint32_t raw[16], xp[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = ldg16(src + 8 * i);
      raw[4 * i] = v.x; raw[4 * i + 1] = v.y; raw[4 * i + 2] = v.z; raw[4 * i + 3] = v.w;
    }
    pair_activations(raw, xp);
    const float sum = bf16_pair_sum(raw);
    acc += fmaf(bf16_to_f32(seg.s[g]), q4_dot_bf16(w, xp) - 128.0f * sum, bf16_to_f32(seg.b[g]) * sum);
  }
  return round_bf16(wave_sum_all(acc));
}

struct PoolDev {
  const uint8_t* base;
  uint64_t header;
  uint64_t stride;
  uint64_t off[9];
  uint32_t records;
};

__device__ __forceinline__ void keep_proj(ProjPtrs& q) {
  VM_KEEP(q.w);
  VM_KEEP(q.s);
  VM_KEEP(q.b);
}

// Local SGPR copy of parts [FIRST, FIRST + PARTS) of a pool view (VM_KEEP).
template <int FIRST, int PARTS>
__device__ __forceinline__ void keep_view(PoolDev& v) {
  VM_KEEP(v.base);
  VM_KEEP(v.header);
  VM_KEEP(v.stride);
  VM_KEEP(v.records);
#pragma unroll
  for (int i = 0; i < PARTS; ++i) VM_KEEP(v.off[FIRST + i]);
}

__device__ __forceinline__ void record_parts(const PoolDev& view, uint32_t record, int proj, ProjPtrs& out) {
  const uint8_t* rec = view.base + view.header + static_cast<uint64_t>(record) * view.stride;
  out.w = reinterpret_cast<const uint32_t*>(rec + view.off[3 * proj + 0]);
  out.s = reinterpret_cast<const uint16_t*>(rec + view.off[3 * proj + 1]);
  out.b = reinterpret_cast<const uint16_t*>(rec + view.off[3 * proj + 2]);
}

// Where a route word points.  With a slot table the word is an expert id
// mapped to a pool slot; otherwise a word with the slot bit is a pool slot,
// and a plain word is a record of the stream view when one is given, else a
// dense expert index.
enum : int { kSrcNone = 0, kSrcPool = 1, kSrcStream = 2, kSrcDense = 3 };

__device__ __forceinline__ int resolve_word(uint32_t word, const int32_t* slot_table, uint32_t experts,
                                            const PoolDev& pool, const PoolDev* stream, bool has_dense,
                                            uint32_t& index) {
  if (slot_table != nullptr) {
    if (word >= experts) return kSrcNone;
    const int32_t slot = slot_table[word];
    if (slot < 0 || static_cast<uint32_t>(slot) >= pool.records) return kSrcNone;
    index = static_cast<uint32_t>(slot);
    return kSrcPool;
  }
  if (word & kSlotBit) {
    index = word & ~kSlotBit;
    return pool.base != nullptr && index < pool.records ? kSrcPool : kSrcNone;
  }
  index = word;
  if (stream != nullptr && stream->base != nullptr) return word < stream->records ? kSrcStream : kSrcNone;
  return has_dense && word < experts ? kSrcDense : kSrcNone;
}

// Pointers of projection `proj` (0 gate, 1 up, 2 down; rows x in_width) of a
// resolved source.
__device__ __forceinline__ void source_proj(int kind, uint32_t index, const PoolDev& pool, const PoolDev* stream,
                                            const ProjPtrs& dense, int proj, uint32_t rows, uint32_t in_width,
                                            ProjPtrs& out) {
  if (kind == kSrcPool) {
    record_parts(pool, index, proj, out);
  } else if (kind == kSrcStream) {
    record_parts(*stream, index, proj, out);
  } else if (kind == kSrcDense) {
    const size_t words = static_cast<size_t>(rows) * (in_width / 8);
    const size_t meta = static_cast<size_t>(rows) * (in_width / kGroup);
    out.w = dense.w + static_cast<size_t>(index) * words;
    out.s = dense.s + static_cast<size_t>(index) * meta;
    out.b = dense.b + static_cast<size_t>(index) * meta;
  }
}

// Resolve the projection `proj` of one route word.  Returns false (and
// leaves `out` untouched) when the word addresses nothing.
__device__ __forceinline__ bool resolve_proj(uint32_t word, const int32_t* slot_table,
                                             uint32_t experts, const PoolDev& pool,
                                             const ProjPtrs& dense, int proj, uint32_t rows,
                                             uint32_t in_width, ProjPtrs& out,
                                             const PoolDev* stream = nullptr) {
  uint32_t index = 0;
  const int kind = resolve_word(word, slot_table, experts, pool, stream, dense.w != nullptr, index);
  if (kind == kSrcNone) return false;
  source_proj(kind, index, pool, stream, dense, proj, rows, in_width, out);
  return true;
}

}  // namespace vm

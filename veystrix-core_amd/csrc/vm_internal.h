// Host-side launch parameters shared between the C ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vm_common.h"

namespace vm {

struct GateUpLaunch {
  const void* x;               // [T, H]
  const uint32_t* routes;      // [T, K] route words (or expert ids with slot_table)
  const int32_t* slot_table;   // optional
  ProjPtrs gate, up;           // dense routed experts
  ProjPtrs shared_gate, shared_up;  // dense shared expert (pair j == K), optional
  PoolDev pool;
  PoolDev stream;              // records for routes without the slot bit, optional
  void* act;                   // [T, S, I], S = K + has_shared
  void* gate_out;              // optional [T, K, I]
  void* up_out;                // optional [T, K, I]
  uint32_t* status;
  uint32_t tokens, slots, hidden, inter, experts, has_shared;
  int act_dtype;
};

struct DownLaunch {
  const void* act;             // [T, S, I]
  const uint32_t* routes;      // [T, K]
  const int32_t* slot_table;
  ProjPtrs down;
  ProjPtrs shared_down;        // internal shared expert (slot K) when has_shared
  const void* shared_sig;      // [T] sigmoid(shared gate), activation dtype
  PoolDev pool;
  PoolDev stream;
  const void* scores;          // [T, K] or null -> per-slot outputs
  int score_dtype;
  const void* shared_y;        // [T, H]
  const void* shared;          // [T, H]
  const void* shared_gate;     // [T]
  void* out;
  uint32_t* status;
  uint32_t tokens, slots, hidden, inter, experts, has_shared;
  int act_dtype;
};

struct RouterLaunch {
  const void* x;               // [T, H]
  const uint16_t* weight;      // [E, H] bf16
  const float* bias;           // optional [E]
  int32_t* inds;               // [T, K]
  void* scores;                // [T, K] activation dtype
  void* gates;                 // optional [T, E]
  float* logits;               // workspace [T, E]
  uint32_t* counter;           // workspace, zero between launches
  // optional shared expert gate (H -> 1 Q4 projection) computed by one extra block
  ProjPtrs seg;
  void* shared_sig;            // [T] activation dtype
  uint32_t tokens, hidden, experts, top_k;
  int act_dtype;
  float blend;
};

hipError_t launch_gateup(const GateUpLaunch& p, hipStream_t stream);
hipError_t launch_down(const DownLaunch& p, hipStream_t stream);
hipError_t launch_router(const RouterLaunch& p, hipStream_t stream);
hipError_t launch_weighted_combine(const void* values, const void* scores, void* out, uint32_t tokens,
                                   uint32_t slots, uint32_t hidden, int act_dtype, int score_dtype,
                                   hipStream_t stream);

// Shape support of the decode kernels.
bool gateup_supported(uint32_t hidden);
bool down_supported(uint32_t inter, uint32_t slots_total, int act_dtype);

// Kernel timing hooks (api.cpp).
void timing_begin(const char* family, hipStream_t stream);
void timing_end(const char* family, hipStream_t stream);

}  // namespace vm

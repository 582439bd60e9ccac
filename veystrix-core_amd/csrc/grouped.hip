// Batched decode / chunked prefill path (token-by-expert grouping).
#include <hip/hip_runtime.h>

#include "../../include/veymoe.h"
#include "vm_internal.h"

extern "C" {

uint64_t vm_moe_grouped_workspace(uint32_t tokens, uint32_t top_k, uint32_t hidden_size, uint32_t inter_size,
                                  uint32_t expert_count, uint32_t act_dtype) {
  (void)tokens; (void)top_k; (void)hidden_size; (void)inter_size; (void)expert_count; (void)act_dtype;
  return 0;
}

int vm_moe_grouped(const VmGroupedArgs* a, void* stream) {
  (void)a; (void)stream;
  return VM_EUNSUPPORTED;
}

}  // extern "C"

// Gather instantiations of the fused row quantizer (truncation: output row t
// reads source row gather[t]; nq_quantize with a gather list).
#include "nq_quant_kernel.h"

namespace nq {

hipError_t dispatch_quant_gather(int head_dim, int L, bool key, int dt, const QuantArgs& a, const QuantTables& t,
                                 hipStream_t s) {
    return dispatch_quant<kSelGather>(head_dim, L, key, dt, a, t, s);
}

}  // namespace nq

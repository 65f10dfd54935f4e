// Row-list instantiations of the fused row quantizer (mask eviction that reads
// and quantizes only the kept rows; nq_quantize with an `order` list).
#include "nq_quant_kernel.h"

namespace nq {

hipError_t dispatch_quant_list(int head_dim, int L, bool key, int dt, const QuantArgs& a, const QuantTables& t,
                               hipStream_t s) {
    return dispatch_quant<kSelList>(head_dim, L, key, dt, a, t, s);
}

}  // namespace nq

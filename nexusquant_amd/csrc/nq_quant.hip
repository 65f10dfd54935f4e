// Entry points of the fused row quantizer (nq_quantize, nq_page_encode) and
// their plain and page instantiations; the kernel is in nq_quant_kernel.h.
#include "nq_quant_kernel.h"

extern "C" int nq_quantize(const nq_quant_desc* d, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(d != nullptr, "nq_quantize: desc is NULL");
    NQ_CHECK_ARG(d->n_tensors >= 0 && d->n_tensors <= 65535, "nq_quantize: n_tensors %d out of range", d->n_tensors);
    if (d->n_tensors == 0) return NQ_OK;
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 96 || d->head_dim == 128 || d->head_dim == 256,
                 "nq_quantize: head_dim %d unsupported by this entry point (64, 96, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(d->levels == 2 || d->levels == 4 || d->levels == 8 || d->levels == 16,
                 "nq_quantize: levels must be 2, 4, 8 or 16 (got %d)", d->levels);
    NQ_CHECK_ARG(d->dtype == NQ_F16 || d->dtype == NQ_BF16 || d->dtype == NQ_F32,
                 "nq_quantize: unknown dtype %d", d->dtype);
    NQ_CHECK_ARG(d->batch > 0 && d->heads > 0 && d->seq_in >= 0 && d->seq_out >= 0,
                 "nq_quantize: bad geometry");
    NQ_CHECK_ARG(d->gather != nullptr || d->seq_out == d->seq_in,
                 "nq_quantize: seq_out must equal seq_in without a gather list");
    NQ_CHECK_ARG(d->src != nullptr, "nq_quantize: src is NULL");
    NQ_CHECK_ARG(d->keep_mode == NQ_KEEP_ZERO || d->keep_mode == NQ_KEEP_WRITE_KEPT ||
                     d->keep_mode == NQ_KEEP_WRITE_EVICTED,
                 "nq_quantize: keep_mode %d unknown", d->keep_mode);
    NQ_CHECK_ARG(d->keep_mode == NQ_KEEP_ZERO || d->keep != nullptr,
                 "nq_quantize: keep_mode %d needs a keep list", d->keep_mode);
    NQ_CHECK_ARG(d->order == nullptr || (d->keep_mode == NQ_KEEP_ZERO && d->keep != nullptr &&
                                         d->n_kept != nullptr && d->gather == nullptr),
                 "nq_quantize: a row list takes keep_mode NQ_KEEP_ZERO, a keep list and n_kept, and no gather");
    const uint64_t rows = (uint64_t)d->batch * d->heads * d->seq_out;
    NQ_CHECK_ARG(rows < (1ull << 31), "nq_quantize: %llu rows per tensor exceeds 2^31", (unsigned long long)rows);
    if (rows == 0) return NQ_OK;
    NQ_CHECK_ARG((d->rope_sin_minus_cos == nullptr) == (d->rope_cos_plus_sin == nullptr),
                 "nq_quantize: give both or neither of rope_sin_minus_cos / rope_cos_plus_sin");
    NQ_CHECK_ARG(d->rope_sin_minus_cos == nullptr || d->head_dim != 96,
                 "nq_quantize: head_dim 96 keys take cos / sin tables only");
    if (d->is_key) {
        NQ_CHECK_ARG(d->rope_cos && d->rope_sin, "nq_quantize: keys need RoPE tables");
        NQ_CHECK_ARG(d->rope_n_pos >= d->seq_in && d->rope_n_pos >= d->seq_out,
                     "nq_quantize: RoPE table has %lld positions, need %d",
                     (long long)d->rope_n_pos, d->seq_in > d->seq_out ? d->seq_in : d->seq_out);
    }
    QuantTables t = {};
    t.src = d->src;
    t.recon = d->recon;
    t.syms = d->syms;
    t.cosets = d->cosets;
    t.scales = d->scales;
    QuantArgs a = {};
    a.gather = d->gather;
    a.keep = d->keep;
    a.order = d->order;
    a.n_kept = d->n_kept;
    a.rope_cos = d->rope_cos;
    a.rope_sin = d->rope_sin;
    a.rope_dm = d->rope_sin_minus_cos;
    a.rope_dp = d->rope_cos_plus_sin;
    a.heads = (uint32_t)d->heads;
    a.seq_in = (uint32_t)d->seq_in;
    a.seq_out = (uint32_t)d->seq_out;
    a.hscale = d->hadamard_scale;
    a.keep_mode = d->keep_mode;
    a.n_tensors = (uint32_t)d->n_tensors;
    a.batch = (uint32_t)d->batch;
    const uint64_t work = plan_work(a, (uint64_t)(d->seq_out + 63) / 64, d->is_key ? kKeyGroup : kMaxGroup,
                                    d->is_key && d->gather ? kGatherKeyMinBlocks : kMinBlocks);
    NQ_CHECK_ARG(work + 8 <= max_blocks(256), "nq_quantize: %llu work items exceed the grid limit",
                 (unsigned long long)work);
    hipStream_t s = (hipStream_t)stream;
    const bool key = d->is_key != 0;
    const hipError_t e = a.order    ? dispatch_quant_list(d->head_dim, d->levels, key, d->dtype, a, t, s)
                         : a.gather ? dispatch_quant_gather(d->head_dim, d->levels, key, d->dtype, a, t, s)
                                    : dispatch_quant<kSelNone>(d->head_dim, d->levels, key, d->dtype, a, t, s);
    NQ_CHECK_HIP(e);
    return NQ_OK;
}

// ------------------------------------------------------- page encoding ----

namespace nq {

template <int D, int L, bool K>
static hipError_t page_dtype(int dt, const QuantArgs& a, const QuantTables& t, hipStream_t s) {
    switch (dt) {
        case NQ_F16: return launch_quant<D, L, K, NQ_F16, D, true>(a, t, s);
        case NQ_BF16: return launch_quant<D, L, K, NQ_BF16, D, true>(a, t, s);
        default: return launch_quant<D, L, K, NQ_F32, D, true>(a, t, s);
    }
}

template <int D>
static hipError_t page_levels(int L, bool key, int dt, const QuantArgs& a, const QuantTables& t, hipStream_t s) {
    switch (L) {
        case 4: return key ? page_dtype<D, 4, true>(dt, a, t, s) : page_dtype<D, 4, false>(dt, a, t, s);
        case 8: return key ? page_dtype<D, 8, true>(dt, a, t, s) : page_dtype<D, 8, false>(dt, a, t, s);
        default: return key ? page_dtype<D, 16, true>(dt, a, t, s) : page_dtype<D, 16, false>(dt, a, t, s);
    }
}

}  // namespace nq

extern "C" int nq_page_encode(const nq_page_desc* d, void* stream) {
    using namespace nq;
    NQ_CHECK_ARG(d != nullptr, "nq_page_encode: desc is NULL");
    NQ_CHECK_ARG(d->n_pages >= 0 && d->n_pages <= 65535, "nq_page_encode: n_pages %d out of range", d->n_pages);
    if (d->n_pages == 0) return NQ_OK;
    NQ_CHECK_ARG(d->head_dim == 64 || d->head_dim == 128 || d->head_dim == 256,
                 "nq_page_encode: head_dim %d unsupported (64, 128, 256)", d->head_dim);
    NQ_CHECK_ARG(d->levels == 4 || d->levels == 8 || d->levels == 16,
                 "nq_page_encode: levels must be 4, 8 or 16 (bits 2, 3, 4; got %d)", d->levels);
    NQ_CHECK_ARG(d->dtype == NQ_F16 || d->dtype == NQ_BF16 || d->dtype == NQ_F32,
                 "nq_page_encode: unknown dtype %d", d->dtype);
    NQ_CHECK_ARG(d->heads > 0 && d->tokens >= 0, "nq_page_encode: bad geometry");
    NQ_CHECK_ARG(d->src && d->codes && d->scales, "nq_page_encode: src, codes and scales are required");
    const uint64_t rows = (uint64_t)d->heads * d->tokens;
    NQ_CHECK_ARG(rows < (1ull << 31), "nq_page_encode: %llu rows per page exceeds 2^31",
                 (unsigned long long)rows);
    if (rows == 0) return NQ_OK;
    NQ_CHECK_ARG((d->rope_sin_minus_cos == nullptr) == (d->rope_cos_plus_sin == nullptr),
                 "nq_page_encode: give both or neither of rope_sin_minus_cos / rope_cos_plus_sin");
    if (d->is_key) {
        NQ_CHECK_ARG(d->positions != nullptr, "nq_page_encode: keys need positions");
        NQ_CHECK_ARG(d->rope_cos && d->rope_sin && d->rope_n_pos > 0 && d->rope_n_pos < (1ll << 31),
                     "nq_page_encode: keys need RoPE tables");
    }
    QuantTables t = {};
    t.src = d->src;
    t.positions = d->positions;
    t.codes8 = d->codes;
    t.scales16 = d->scales;
    QuantArgs a = {};
    a.rope_cos = d->rope_cos;
    a.rope_sin = d->rope_sin;
    a.rope_dm = d->rope_sin_minus_cos;
    a.rope_dp = d->rope_cos_plus_sin;
    a.heads = 1u;  // a page's (head, token) rows are one flat run of rows
    a.seq_in = a.seq_out = (uint32_t)rows;
    a.hscale = d->hadamard_scale;
    a.keep_mode = NQ_KEEP_ZERO;
    a.n_tensors = (uint32_t)d->n_pages;
    a.batch = 1u;
    a.page_tokens = (uint32_t)(d->tokens > 0 ? d->tokens : 1);
    a.rope_n_pos = (uint32_t)(d->is_key ? d->rope_n_pos : 1);
    const uint64_t work = plan_work(a, (rows + 63) / 64, kMaxGroup);
    NQ_CHECK_ARG(work + 8 <= max_blocks(256), "nq_page_encode: %llu work items exceed the grid limit",
                 (unsigned long long)work);
    hipStream_t s = (hipStream_t)stream;
    const bool key = d->is_key != 0;
    hipError_t e;
    switch (d->head_dim) {
        case 64: e = page_levels<64>(d->levels, key, d->dtype, a, t, s); break;
        case 128: e = page_levels<128>(d->levels, key, d->dtype, a, t, s); break;
        default: e = page_levels<256>(d->levels, key, d->dtype, a, t, s); break;
    }
    NQ_CHECK_HIP(e);
    return NQ_OK;
}

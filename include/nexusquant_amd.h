/*
 * nexusquant_amd -- C ABI of the MI355X (gfx950) KV-cache compression library.
 *
 * Every entry point is asynchronous on the HIP stream it is given, borrows the
 * device pointers it is passed (no ownership transfer), allocates nothing, and
 * returns 0 on success or a negative NQ_E* code; nq_last_error() then holds a
 * message for the calling thread.  Tensors are row-major and contiguous.
 *
 * The reference (jagmarques/nexusquant v0.5.0) is pure Python/PyTorch; these
 * entry points replace the torch operator sequences cited on each declaration.
 */
#ifndef NEXUSQUANT_AMD_H
#define NEXUSQUANT_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NQ_ABI_VERSION 8

/* status codes */
#define NQ_OK 0
#define NQ_EINVAL -1      /* bad argument (shape, levels, pointer) */
#define NQ_EUNSUPPORTED -2 /* valid request this build does not implement */
#define NQ_EHIP -3        /* HIP runtime error (launch, device) */

/* what nq_quantize does with rows whose keep entry is 0 */
#define NQ_KEEP_ZERO 0
#define NQ_KEEP_WRITE_KEPT 1
#define NQ_KEEP_WRITE_EVICTED 2

/* element types of input tensors */
#define NQ_F16 0
#define NQ_BF16 1
#define NQ_F32 2

/*
 * One fused quantizer launch over n_tensors tensors of identical geometry
 * [batch, heads, seq_in, head_dim] and identical role (keys or values).
 *
 * Per row (one head vector of one token): optional inverse RoPE at the row's
 * source position, zero-pad to the next power of two D, Walsh-Hadamard, per-row
 * amax scale, relaxed-E8 nearest point at `levels` (2, 4, 8, 16), clamp; then
 * write any of
 *   recon  [batch, heads, seq_out, head_dim] fp16: inverse Hadamard, rescale,
 *          forward RoPE at the output position (the reference's drop-in output);
 *   syms   [batch, heads, seq_out, D/8 * bits] packed symbols (bits = 2,3,4,5
 *          for levels 2,4,8,16);
 *   cosets [batch, heads, seq_out, D/64] coset bitmaps;
 *   scales [batch, heads, seq_out] fp32 row scales.
 * Row selection: output row t of batch b reads source token gather[b*seq_out+t]
 * (truncation) or token t (gather == NULL, then seq_out == seq_in).  With a
 * keep list, keep_mode says what happens to rows whose keep[b*seq_in + src]
 * is 0: NQ_KEEP_ZERO zeroes them before quantization (mask eviction);
 * NQ_KEEP_WRITE_KEPT writes only the rows with keep != 0 and
 * NQ_KEEP_WRITE_EVICTED only the rows with keep == 0, leaving the other rows
 * of every output untouched (soft eviction: two launches, kept rows at the
 * layer's levels and evicted rows at levels 2, into the same outputs).
 * RoPE tables are fp32 [rope_n_pos, head_dim/2]; keys use row position
 * src (inverse) and t (forward).  For power-of-two head dims the kernel
 * folds the rotation into the top Hadamard stage, whose pairs (i, i + d/2)
 * are the RoPE pairs; it then needs fl(sin - cos) and fl(cos + sin), which it
 * reads from rope_sin_minus_cos / rope_cos_plus_sin when given (same layout)
 * and otherwise forms from rope_cos / rope_sin.  Either way the results are
 * identical; the precomputed tables save two operations per pair.
 *
 * Row lists (mask eviction without work on evicted rows): with keep_mode
 * NQ_KEEP_ZERO, a keep list and order != NULL (then n_kept != NULL, gather ==
 * NULL, seq_out == seq_in), order[b*seq_in .. +seq_in) is a permutation of the
 * row's positions with its n_kept[b] kept positions first, as nq_keep_mask
 * writes kept_idx.  The kept positions are quantized and written at their own
 * positions; the evicted ones are not read, and get the outputs a zeroed row
 * has (recon 0, every symbol L/2, coset bits 0, scale 1e-8 * 2/L: the
 * reference's amax clamp).  The outputs equal those of the same call without
 * order, bit for bit, up to the sign of zero in recon.
 *
 * Replaces (keep_mode 1 + 2): the soft-eviction loop   pipeline.py:1129-1183
 *
 * Replaces: NexusQuantQuantOnly.compress            pipeline.py:232-265
 *           NexusQuantEvict.compress (hard path)     pipeline.py:1190-1242
 *           NexusQuantEvictTruncate.compress (loop)  pipeline.py:1343-1397
 *           E8Lattice.quantize_perhead / nearest_point  e8_lattice.py:27-124
 *           inverse_rope / forward_rope (+_at_positions) rope_utils.py:75-249
 *           the dense Hadamard einsums               pipeline.py:250,253,258,261
 *           VLLM code format (int8 2p + scale)       vllm_backend.py:267-338
 */
typedef struct nq_quant_desc {
    int32_t n_tensors;
    int32_t batch, heads, seq_in, seq_out, head_dim;
    int32_t dtype;          /* NQ_F16 / NQ_BF16 / NQ_F32 */
    int32_t levels;         /* 2, 4, 8 or 16 */
    int32_t is_key;         /* 1: inverse/forward RoPE around the quantizer */
    int32_t keep_mode;      /* NQ_KEEP_ZERO / NQ_KEEP_WRITE_KEPT / NQ_KEEP_WRITE_EVICTED */
    /* device arrays of n_tensors base addresses (uint64); recon/syms/cosets/
     * scales arrays may be NULL to skip that output */
    const uint64_t* src;
    const uint64_t* recon;
    const uint64_t* syms;
    const uint64_t* cosets;
    const uint64_t* scales;
    const int32_t* gather;  /* device [batch * seq_out] or NULL */
    const uint8_t* keep;    /* device [batch * seq_in] or NULL */
    const float* rope_cos;  /* device [rope_n_pos, head_dim/2] (keys) */
    const float* rope_sin;
    int64_t rope_n_pos;
    float hadamard_scale;   /* h_D of the reference's Sylvester matrix */
    float reserved_f;
    const float* rope_sin_minus_cos;  /* optional, [rope_n_pos, head_dim/2]; NULL: formed in-kernel */
    const float* rope_cos_plus_sin;
    const int32_t* order;   /* device [batch * seq_in] row list (kept first) or NULL */
    const int32_t* n_kept;  /* device [batch]: kept entries at the head of each order row */
} nq_quant_desc;

int nq_quantize(const nq_quant_desc* desc, void* stream);

/*
 * Key-key importance (SnapKV-style proxy): keys [batch, heads, seq, head_dim]
 * (dtype NQ_F16/NQ_BF16/NQ_F32, head_dim 64/96/128/256); queries are the last
 * obs = min(obs_window, seq) keys; importance[batch, seq] = mean over heads of
 * the per-key sum over queries of softmax(q . k * scale) over all keys, in
 * fp32.  scale is the reference's fp32 d**-0.5.  workspace: device buffer of
 * at least nq_score_keykey_workspace(batch, heads, seq, obs_window) bytes
 * (caller owned; per-split row statistics and per-head column sums).
 *
 * Replaces: NexusQuantEvict._score_importance          pipeline.py:756-782
 */
int64_t nq_score_keykey_workspace(int32_t batch, int32_t heads, int32_t seq, int32_t obs_window);
int nq_score_keykey(const void* keys, int32_t dtype, int32_t batch, int32_t heads, int32_t seq,
                    int32_t head_dim, int32_t obs_window, float scale, float* importance, void* workspace,
                    int64_t workspace_bytes, void* stream);

/*
 * nq_score_keykey without a workspace argument: the partial row statistics
 * live in a static device array of the library, NQ_KEYKEY_SCRATCH_BYTES per
 * GPU (held from library load until the process ends), so the call allocates
 * nothing -- no hipMalloc, no hipFree, no allocating library call.  Shapes
 * whose nq_score_keykey_workspace(batch, heads, seq, obs_window) exceeds the
 * scratch return NQ_EINVAL before any launch (8 MiB covers e.g. 64 heads x
 * 131072 tokens with 64 observation queries).  The stream must belong to the
 * current device.  Every call on a GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other threads) race.
 *
 * No counterpart in the reference: this entry point is for callers that
 * cannot allocate -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.
 */
#define NQ_KEYKEY_SCRATCH_BYTES (8 << 20)
int nq_score_keykey_noalloc(const void* keys, int32_t dtype, int32_t batch, int32_t heads, int32_t seq,
                            int32_t head_dim, int32_t obs_window, float scale, float* importance, void* stream);

/*
 * Real-attention importance of one layer, accumulated: importance[b, j] +=
 * mean over q_heads of sum_i p[b, h, i, j], with
 * p = round(softmax_fp32(f(round(round(q . k) * scaling)))) under the causal
 * mask, round = rounding to the model dtype (fp16/bf16; none for fp32) as
 * transformers' eager attention does; query head h reads key head
 * h / (q_heads / kv_heads).  q [batch, q_heads, seq, head_dim],
 * k [batch, kv_heads, seq, head_dim], both post-RoPE.
 * sliding_window > 0: query i sees keys i - sliding_window < j <= i only
 * (transformers' sliding_window_overlay); 0: plain causal.
 * logit_map (fp16/bf16 only; NULL: f = identity): 65536 entries, the bits of
 * f(x) at the model-dtype bits of x, for an elementwise logit transform f that
 * is monotone non-decreasing -- Gemma-2's soft-capping
 * round(round(tanh(round(x / cap))) * cap), built by the host with the
 * framework's own ops.  workspace: at least
 * nq_score_real_workspace(batch, q_heads, seq) bytes (caller owned).
 *
 * Replaces: NexusQuantEvict._score_importance_real   pipeline.py:784-836
 *           (eager_attention_forward + repeat_kv, transformers 5.15.0
 *            models/llama/modeling_llama.py:179-213; soft-capping
 *            models/gemma2/modeling_gemma2.py:184-215; the sliding-window
 *            mask masking_utils.py:92-101)
 */
int64_t nq_score_real_workspace(int32_t batch, int32_t q_heads, int32_t seq);
int nq_score_real(const void* q, const void* k, int32_t dtype, int32_t batch, int32_t q_heads,
                  int32_t kv_heads, int32_t seq, int32_t head_dim, float scaling, int32_t sliding_window,
                  const uint16_t* logit_map, float* importance, void* workspace, int64_t workspace_bytes,
                  void* stream);

/*
 * The scoring pass's attention output without materialising P: the row
 * statistics and (importance != NULL) the column sums of nq_score_real, then
 * out = round_T(P V) [batch, q_heads, seq, head_dim] with P = round_T(softmax_fp32
 * (round_T(round_T(Q K^T) * scaling))), causal, query head h reading kv head
 * h / (q_heads / kv_heads) -- eager_attention_forward's arithmetic, P V summed
 * in fp32 on the matrix cores.  fp16 / bf16, head_dim 64 or 128, 16-byte aligned
 * tensors; v [batch, kv_heads, seq, head_dim]; sliding_window and logit_map as
 * for nq_score_real.  workspace:
 * nq_attention_real_workspace bytes (row statistics, column sums and V
 * transposed with the keys of each 32-key block in the accumulator's order).
 *
 * Replaces: eager_attention_forward (transformers modeling_llama.py:179-213) in
 *           the scoring forward of _score_importance_real  pipeline.py:784-836
 */
int64_t nq_attention_real_workspace(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t seq, int32_t head_dim);
int nq_attention_real(const void* q, const void* k, const void* v, int32_t dtype, int32_t batch, int32_t q_heads,
                      int32_t kv_heads, int32_t seq, int32_t head_dim, float scaling, int32_t sliding_window,
                      const uint16_t* logit_map, float* importance, void* out, void* workspace,
                      int64_t workspace_bytes, void* stream);

/*
 * Keep mask from importance[batch, seq] (fp32): position 0, the last
 * sliding_window positions, the k most important positions of [1, prefix)
 * (ties at the k-th value keep the lowest positions), and protected_pos.
 * prefix = max(seq - sliding_window, 0) and k = min(n_keep, prefix - 1) are
 * computed by the caller exactly as the reference does (Python double).
 * Writes keep[batch, seq] (0/1), kept_idx[batch, seq] and n_kept[batch]:
 * row b of kept_idx holds its n_kept[b] kept positions ascending, then its
 * evicted positions descending (a permutation of 0 .. seq-1, the row list
 * nq_quantize takes as `order`).
 *
 * Replaces: NexusQuantEvict._build_keep_mask (topk + scatter)  pipeline.py:895-959
 *           keep_mask[0].nonzero() of the truncation path      pipeline.py:1319
 */
int nq_keep_mask(const float* importance, int32_t batch, int32_t seq, int32_t sliding_window,
                 int32_t prefix, int32_t k, const int32_t* protected_pos, int32_t n_protected,
                 uint8_t* keep, int32_t* kept_idx, int32_t* n_kept, void* stream);

/*
 * fp16 passthrough of protected layers: dst[t] = fp16(src[gather[b, t]]) or
 * fp16(src[t]) * keep[b, t], for n_tensors tensors (device arrays of base
 * addresses) of shape [batch, heads, seq_in, head_dim].
 *
 * Replaces: protected-layer branches  pipeline.py:1204-1210 (mask), 1359-1368 (truncate)
 */
int nq_gather_rows(const uint64_t* src, const uint64_t* dst, int32_t n_tensors, int32_t dtype, int32_t batch,
                   int32_t heads, int32_t seq_in, int32_t seq_out, int32_t head_dim, const int32_t* gather,
                   const uint8_t* keep, void* stream);

/*
 * Packed codes of n_tensors tensors [batch, heads, seq, head_dim] written by
 * nq_quantize (syms / cosets / scales arrays of base addresses).
 */
typedef struct nq_codes_desc {
    int32_t n_tensors;
    int32_t batch, heads, seq, head_dim;
    int32_t levels;
    int32_t is_key;          /* dequantize: forward RoPE at positions 0..seq-1 */
    int32_t reserved;
    const uint64_t* syms;
    const uint64_t* cosets;
    const uint64_t* scales;
    const uint64_t* out;     /* per tensor output base address */
    const float* rope_cos;   /* [rope_n_pos, head_dim/2], keys only */
    const float* rope_sin;
    int64_t rope_n_pos;
    float hadamard_scale;
    float reserved_f;
    const float* rope_sin_minus_cos;  /* optional, as in nq_quant_desc */
    const float* rope_cos_plus_sin;
} nq_codes_desc;

/*
 * Codes -> fp16 reconstruction [batch, heads, seq, head_dim]; identical to the
 * reconstruction nq_quantize writes for the same rows.
 *
 * Replaces: _dequantize_perhead + inverse Hadamard + forward_rope
 *           vllm_backend.py:319-338, pipeline.py:253-255
 */
int nq_dequantize(const nq_codes_desc* desc, void* stream);

/*
 * Codes -> int8 code = 2p per coordinate [batch, heads, seq, D] (delta = 0), or
 * the temporal delta stream of those codes along tokens, first token raw,
 * int8 wrap (delta = 1).
 *
 * Replaces: _quantize_perhead_with_scales code output  vllm_backend.py:309-314
 *           _compress_with_delta_zstd delta step        compression_accounting.py:56-60
 */
int nq_codes_to_int8(const nq_codes_desc* desc, int32_t delta, void* stream);

/*
 * Token deltas of raw int8 rows: out[s, 0, :] = x[s, 0, :] and
 * out[s, t, :] = x[s, t, :] - x[s, t-1, :] (int8 wrap) for n_tensors tensors
 * of `streams` x seq x coords int8 (any coords > 0).  Addresses are aligned to
 * 16 bytes when coords % 16 == 0, to 4 when coords % 4 == 0; out must not
 * overlap src.  At most 2^32 - 2^22 words of 16, 4 or 1 bytes per tensor.
 *
 * Replaces: temporal_delta_encode  temporal_codec.py:30-52
 */
int nq_delta_encode(const uint64_t* src, const uint64_t* out, int32_t n_tensors, int32_t streams, int32_t seq,
                    int32_t coords, void* stream);

/*
 * Inverse of the delta stream: out[s, t, :] = sum_{u <= t} deltas[s, u, :]
 * (int8 wrap) for n_tensors tensors of `streams` x seq x coords int8 (any
 * coords > 0, alignment as for nq_delta_encode).  out may equal deltas (in
 * place) but must not partially overlap it.  Few columns are scanned in token
 * chunks (three launches, chunk totals staged in out), many in one launch.
 *
 * Replaces: _decompress_with_delta cumsum  compression_accounting.py:70-77
 *           temporal_delta_decode          temporal_codec.py:55-73
 */
int nq_delta_decode(const uint64_t* deltas, const uint64_t* out, int32_t n_tensors, int32_t streams, int32_t seq,
                    int32_t coords, void* stream);

/*
 * Merge eviction, run before the hard-eviction quantizer: for each batch row,
 * every evicted token's value is added into the kept token whose value
 * centroid is most similar (cosine, first on ties), weighted by
 * w = fp32(imp_e / (imp_s + imp_e + 1e-8)) (double arithmetic), over the
 * n_tensors value tensors [batch, heads, seq, head_dim] (heads <= 256) of
 * the layers whose seq equals the mask's.  Centroids are the fp32 means over
 * heads, averaged over those layers; merged rows accumulate
 * v_s = fl(v_s + fl(w_e v_e)) over their evicted tokens in ascending order and
 * are rounded once to the tensor type; every other row is copied.  keep /
 * kept_idx / n_kept are nq_keep_mask's outputs.  Optional outputs: the
 * centroids, and survivor [batch, seq] (the survivor position of each
 * evicted position, -1 at kept positions).  workspace: nq_merge_workspace
 * bytes (caller owned).
 *
 * Replaces: NexusQuantEvict._apply_merge_eviction  pipeline.py:961-1048
 */
typedef struct nq_merge_desc {
    int32_t n_tensors;
    int32_t batch, heads, seq, head_dim;
    int32_t dtype;               /* NQ_F16 / NQ_BF16 / NQ_F32 */
    const uint64_t* src;         /* value tensors (device array of addresses) */
    const uint64_t* dst;         /* merged outputs, same shape and type; must not alias src */
    const uint8_t* keep;         /* [batch, seq] */
    const int32_t* kept_idx;     /* [batch, seq] */
    const int32_t* n_kept;       /* [batch] */
    const float* importance;     /* [batch, seq] */
    float* centroids;            /* optional [batch, seq, head_dim] */
    int32_t* survivor;           /* optional [batch, seq] */
    void* workspace;
    int64_t workspace_bytes;
} nq_merge_desc;

int64_t nq_merge_workspace(int32_t batch, int32_t seq, int32_t head_dim);
int nq_merge_values(const nq_merge_desc* desc, void* stream);

/*
 * Chunked rANS coding of int8 lattice codes c = 2p (|c| <= levels).  The coder
 * is the reference's: 32-bit state in [2^16, 2^32), 16-bit renormalisation,
 * frequencies summing to 4096, symbols s = c + levels (alphabet 2 levels + 1)
 * when half-integer points occur (has_half), else s = c/2 + levels/2 (alphabet
 * levels + 1).  The n codes are cut into chunks of `chunk` symbols, each coded
 * on its own from the initial state, so chunk k's words equal the reference
 * encoder's output for that chunk's symbols.
 *   nq_rans_histogram: hist[2 levels + 1] += counts of c + levels (uint32,
 *     caller-zeroed); codes 16-byte aligned; at most 2^32 - 1 codes per call,
 *     so that no bin wraps (count a longer stream in pieces).
 *   nq_rans_encode: per chunk, words right-aligned in scratch
 *     (nq_rans_scratch_words(n, chunk) uint16), their counts in n_words
 *     [n_chunks], and offset [n_chunks + 1] = exclusive scan of the counts;
 *     codes 16-byte and scratch 8-byte aligned.
 *   nq_rans_compact: words[offset[k] ..] = chunk k's words; scratch 8-byte
 *     and words 4-byte aligned.
 *   nq_rans_decode: codes from the compacted words and offsets; words 8-byte
 *     and codes 16-byte aligned.  offset must be a layout nq_rans_encode can
 *     write: offset[0] = 0, non-decreasing, chunk k holding at most its symbol
 *     count + 2 words, and words[0 .. offset[n_chunks]) readable (the kernel
 *     reads ahead of a chunk's words up to that end).  A stream from elsewhere
 *     is checked on the host first (entropy.check_stream_layout).
 * freq: uint16 [alphabet], summing to 4096, nonzero for every symbol present.
 *
 * Replaces: _build_freq_table / _rans_encode / _rans_decode use in
 *           encode_e8 / decode_e8   entropy_coder.py:163-345, 376-484
 *           (the reference codes one sequential stream on the host)
 */
int nq_rans_histogram(const int8_t* codes, int64_t n, int32_t levels, uint32_t* hist, void* stream);
int64_t nq_rans_scratch_words(int64_t n, int32_t chunk);
int nq_rans_encode(const int8_t* codes, int64_t n, int32_t levels, int32_t has_half, const uint16_t* freq,
                   int32_t alphabet, int32_t chunk, uint16_t* scratch, uint32_t* n_words, uint64_t* offset,
                   void* stream);
int nq_rans_compact(const uint16_t* scratch, const uint32_t* n_words, const uint64_t* offset, int64_t n,
                    int32_t chunk, uint16_t* words, void* stream);
int nq_rans_decode(const uint16_t* words, const uint64_t* offset, int64_t n, int32_t levels, int32_t has_half,
                   const uint16_t* freq, int32_t alphabet, int32_t chunk, int8_t* codes, void* stream);

/*
 * Pages of the vLLM compressor: n_pages pages of identical geometry
 * [heads, tokens, head_dim] (head_dim 64, 128 or 256), keys or values, at
 * `levels` 4, 8 or 16 (bits 2, 3, 4).  The format is the reference's
 * CompressedPage: codes int8 [heads, tokens, head_dim] holding 2p for the
 * clamped relaxed-E8 point p of the Hadamard-rotated row, scales fp16
 * [heads, tokens] (the row scale amax / (levels/2) rounded to fp16), and
 * int32 absolute positions [tokens] at which keys carry RoPE.  Arrays are
 * device arrays of n_pages base addresses (uint64).
 */
typedef struct nq_page_desc {
    int32_t n_pages;
    int32_t heads, tokens, head_dim;
    int32_t dtype;           /* nq_page_encode input: NQ_F16 / NQ_BF16 / NQ_F32 */
    int32_t levels;
    int32_t is_key;
    int32_t reserved;
    const uint64_t* src;       /* encode: K or V pages */
    const uint64_t* positions; /* int32 [tokens] per page (keys) */
    const uint64_t* codes;     /* int8 [heads, tokens, head_dim] per page */
    const uint64_t* scales;    /* fp16 [heads, tokens] per page */
    const uint64_t* out;       /* decode: fp16 [heads, tokens, head_dim] per page */
    const float* rope_cos;     /* fp32 [rope_n_pos, head_dim/2], keys */
    const float* rope_sin;
    const float* rope_sin_minus_cos;  /* optional fl(sin - cos) / fl(cos + sin) */
    const float* rope_cos_plus_sin;
    int64_t rope_n_pos;        /* positions must lie in [0, rope_n_pos) */
    float hadamard_scale;
    float reserved_f;
} nq_page_desc;

/*
 * Encode pages: inverse RoPE at each token's absolute position (keys),
 * Walsh-Hadamard, per-row scale, relaxed E8 at `levels`, clamp; writes codes
 * and scales.  Row arithmetic is nq_quantize's.
 *
 * Replaces: NexusQuantKVCompressor.compress_page        vllm_backend.py:344-392
 *           _rope_remove_page / _quantize_perhead_with_scales  :187-224, 267-314
 */
int nq_page_encode(const nq_page_desc* desc, void* stream);

/*
 * Decode pages to fp16 [heads, tokens, head_dim]: x = (code / 2) * scale,
 * inverse Walsh-Hadamard (exact on the integer codes), forward RoPE at the
 * stored positions (keys), rounding to fp16.
 *
 * Replaces: NexusQuantKVCompressor.decompress_page      vllm_backend.py:394-429
 *           _rope_apply_page / _dequantize_perhead       :226-265, 316-338
 */
int nq_page_decode(const nq_page_desc* desc, void* stream);

/*
 * Logits of queries against one page (n_pages == 1): query [heads, q_len,
 * head_dim] of type q_dtype, logits fp32 [heads, q_len, tokens] =
 * (q . k) / scale_divisor with k the page's decoded keys in fp32 (before the
 * fp16 rounding of nq_page_decode).
 *
 * Replaces: NexusQuantKVCompressor.decompress_for_attention  vllm_backend.py:431-467
 */
int nq_page_logits(const nq_page_desc* desc, const void* query, int32_t q_dtype, int32_t q_len,
                   float scale_divisor, float* logits, void* stream);

/*
 * Nibble packing of int8 codes [rows, d]: out[r, j] = n(2j) | n(2j+1) << 4 with
 * n(k) = clamp(code[r, k] + 8, 0, 15) and n(d) = 0 for odd d; packed is
 * [rows, (d + 1) / 2] bytes.  Unpacking reads [rows, packed_cols] bytes and
 * writes the first d <= 2 * packed_cols nibbles of each row minus 8.
 *
 * Replaces: pack_codes_nibble / unpack_codes_nibble   vllm_backend.py:475-536
 */
int nq_nibble_pack(const int8_t* codes, int64_t rows, int32_t d, uint8_t* packed, void* stream);
int nq_nibble_unpack(const uint8_t* packed, int64_t rows, int32_t packed_cols, int32_t d, int8_t* codes,
                     void* stream);

/*
 * Decode attention read straight from compressed pages: for each batch row
 * and query head, softmax(q . k / scale_divisor) . v over the row's tokens,
 * where k and v are the pages' decoded keys (bit for bit nq_page_decode's
 * fp16 keys) and values, query head h reading kv head h / (q_heads /
 * kv_heads).  Output [batch, q_heads, head_dim] has the query's type and
 * holds the fp16-rounded result; rows with no tokens are zero.
 *
 * The caller describes where the tokens are with a chunk plan (device int32
 * arrays; nexusquant_amd/vllm_backend.py builds it):
 *   units        [n_units * 16] unit records, each up to 16 consecutive tokens
 *                of one page (nq_page_desc layout, heads = kv_heads), addressed
 *                at kv head 0 and the unit's first token t0:
 *                  [0..1]  key codes + t0 * head_dim        (uint64 address)
 *                  [2..3]  value codes + t0 * head_dim
 *                  [4..5]  key scales + t0                 (fp16 elements)
 *                  [6..7]  value scales + t0
 *                  [8..9]  positions + t0                  (int32 elements)
 *                  [10]    tokens the page stores per head (its row stride)
 *                  [11]    tokens in the unit (1..16)
 *                  [12]    offset of the unit's first token in its chunk
 *                  [13..15] unused;
 *   chunk_units  [n_chunks + 1] units of each chunk (consecutive);
 *   chunk_row    [n_chunks] batch row of each chunk;
 *   chunk_tokens [n_chunks] tokens of each chunk, at most
 *                nq_paged_attention_chunk_tokens();
 *   row_chunks   [batch + 1] chunks of each row (consecutive, ascending).
 * workspace: nq_paged_attention_workspace(n_chunks, q_heads, head_dim) bytes.
 * q_heads / kv_heads may be 1, 2, 4, or 8 (8 with fp16 queries).
 *
 * Replaces: NexusQuantPagedAttention.forward   vllm_backend.py:692-765
 */
typedef struct nq_attn_desc {
    int32_t batch, q_heads, kv_heads, head_dim;
    int32_t q_dtype;             /* NQ_F16 / NQ_BF16 / NQ_F32 */
    int32_t n_chunks;
    const void* query;           /* [batch, q_heads, head_dim] */
    void* out;                   /* [batch, q_heads, head_dim], q_dtype */
    const int32_t* units;
    const int32_t* chunk_units;
    const int32_t* chunk_row;
    const int32_t* chunk_tokens;
    const int32_t* row_chunks;
    const float* rope_cos;
    const float* rope_sin;
    const float* rope_sin_minus_cos;  /* optional, as in nq_page_desc */
    const float* rope_cos_plus_sin;
    int64_t rope_n_pos;
    float hadamard_scale;
    float scale_divisor;         /* logits = q . k / scale_divisor (fp32 sqrt(head_dim)) */
    void* workspace;
    int64_t workspace_bytes;
} nq_attn_desc;

int32_t nq_paged_attention_chunk_tokens(void);
int64_t nq_paged_attention_workspace(int32_t n_chunks, int32_t q_heads, int32_t head_dim);
int nq_paged_attention(const nq_attn_desc* desc, void* stream);

/*
 * Fused dequantize + matrix product over the standalone E8 code format:
 * out[k, j] = sum_{h < h} (codes[k, h] * scales[k]) * query[h, j] for
 * codes int8 [k_rows, h_pad] (row stride h_pad, 8-byte aligned; columns
 * h .. h_pad-1 are padding and ignored), scales fp32 [k_rows], query fp32
 * [h, q_cols] row-major and out fp32 [k_rows, q_cols].  Requires
 * 0 < h <= h_pad <= 256 and h_pad % 8 == 0.  Computed on bf16 MFMAs with the
 * query split into three bf16 parts: every product is exact, sums are fp32.
 *
 * Replaces: e8_dequant_matmul          nexusquant/kernels/e8_triton.py:613-660
 *           e8_dequant_matmul_kernel   nexusquant/kernels/e8_triton.py:373-444
 */
int nq_e8_dequant_matmul(const int8_t* codes, const float* scales, const float* query, float* out, int64_t k_rows,
                         int32_t h_pad, int32_t h, int32_t q_cols, void* stream);

/*
 * The relaxed-E8 rule on its own: nq_e8_nearest_point maps n_groups fp32
 * 8-groups x to their lattice points (no clamp); nq_e8_quantize_perhead maps
 * each of `rows` fp32 rows of length d to q * scale with scale = max(amax,
 * 1e-8) / (levels / 2) and q the rule applied to the zero-padded 8-groups of
 * x / scale, clamped to +-levels/2.  Integer candidate rint(x) with the first
 * smallest-gap coordinate stepped toward x on an odd sum; half candidate
 * rint(x - 0.5) + 0.5, chosen when its squared distance is smaller.
 * nq_e8_nearest_point needs 16-byte aligned x and out.
 *
 * Replaces: E8Lattice.nearest_point / quantize_perhead   e8_lattice.py:27-69, 97-124
 *           e8_nearest_point / e8_quantize_perhead      nexusquant/kernels/e8_triton.py:455-522
 */
int nq_e8_nearest_point(const float* x, float* out, int64_t n_groups, void* stream);
int nq_e8_quantize_perhead(const float* x, float* out, int64_t rows, int32_t d, int32_t levels, void* stream);

/*
 * Symbol side of the single-stream E8 container (encode_e8 / decode_e8); the
 * rANS chain is nq_rans_encode / nq_rans_decode with one chunk of n_groups * 8
 * symbols.  Groups of 8 coordinates share scales[g], or scales[0] when
 * n_scales == 1.
 *   nq_e8_stream_codes: codes[i] = clip(rint(2 * (quantized[i] / max(s, 1e-8))),
 *     -levels, levels) as int8 (IEEE fp32 division); *has_half is OR-ed with 1
 *     when some rint(2x) is odd before the clip (|x - round(x)| > 0.25).  The
 *     caller zeroes *has_half.  quantized 16-byte aligned, codes 8-byte aligned;
 *     levels 2, 4, 8 or 16.
 *   nq_e8_stream_values: out[i] = (codes[i] / 2) * fp32(scales_f16[g]) (fp32
 *     product); codes 8-byte and out 16-byte aligned.
 *
 * Replaces: encode_e8 symbol mapping  entropy_coder.py:375-386, 35-75
 *           decode_e8 reconstruction  entropy_coder.py:418-420, 78-86
 */
int nq_e8_stream_codes(const float* quantized, const float* scales, int64_t n_groups, int64_t n_scales, int32_t levels,
                       int8_t* codes, uint32_t* has_half, void* stream);
int nq_e8_stream_values(const int8_t* codes, const uint16_t* scales_f16, int64_t n_groups, int64_t n_scales,
                        float* out, void* stream);

/* Library version and the last error message of the calling thread. */
int nq_abi_version(void);
const char* nq_last_error(void);

/*
 * Hash of the sources and compiler flags the library was built from (16 hex
 * digits).  Build provenance, no counterpart in the reference: the Python
 * loader compares it with the sources next to it and refuses a stale build.
 */
const char* nq_source_hash(void);

#ifdef __cplusplus
}
#endif

#endif /* NEXUSQUANT_AMD_H */

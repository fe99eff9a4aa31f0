/*
 * latticequant_amd.h -- C ABI of the MI355X (gfx950) E8 + rANS compressed-KV path.
 *
 * Conventions
 *   - Every pointer argument named d_* is device memory; h_* is host memory.
 *   - Every entry point is stream-ordered on the hipStream_t it receives and
 *     returns an int status (LQ_OK = 0, negative = error, see lq_status_string).
 *   - Nothing here allocates device memory: outputs and workspaces are passed
 *     in by the caller, sized with the *_workspace_size helpers.
 *   - Nothing here synchronises the stream except the functions that say so.
 *   - Geometry of a "chunk" follows CompressedKVCache._compress_tensor
 *     (reference llm/compressed_kv_cache.py:176-287): a (B, H, T, hd) tensor is
 *     n_heads = B*H heads of bph = T*hd/8 contiguous 8-dim vectors.  A batch of
 *     chunks with identical geometry is processed per call; chunk c's input
 *     vectors start at c * n_heads * bph.
 *   - Checkpoint blocks: the stream (coset c, coordinate i) of a chunk is the
 *     reference's rANS stream; its symbols are additionally grouped by vector
 *     block of LQ_BLK vectors so that encode and decode run one block per lane.
 *     The bitstream words themselves are the reference's, bit for bit.
 */
#ifndef LATTICEQUANT_AMD_H
#define LATTICEQUANT_AMD_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LQ_L 1024          /* rANS precision (reference core/gpu_ans.py:44-45) */
#define LQ_BLK 512         /* vectors per checkpoint block */
#define LQ_ESC_MAX_SHIFT 7 /* largest escape shift k_j (lq_chunk_escape_plan) */
#define LQ_SYM_STRIDE 4352 /* symbols per block in the staging layout (8 * LQ_BLK + 2 x 128 padding);
                              bytes: x 1 for int8 symbols, x 2 for the wide (int16) path */
#define LQ_MAXSYM 1028     /* alphabet capacity of a table: the reference's L = 1024 + 4 guard entries */
#define LQ_STREAMS 16      /* 2 cosets x 8 coordinate streams per chunk */

/* status codes */
#define LQ_OK 0
#define LQ_ERR_ARG -1
#define LQ_ERR_LAUNCH -2
#define LQ_ERR_ALPHABET -3     /* alphabet > L=1024: the reference never terminates */
#define LQ_ERR_RANGE -4        /* lattice symbol outside int8 */
#define LQ_ERR_SCRATCH -5      /* request larger than a static scratch array (allocation-free entry points) */

/* per-chunk status bits written by the device */
#define LQ_ST_SYM_OVERFLOW 1   /* a lattice symbol did not fit the staging type (int8: use the wide path) */
#define LQ_ST_ALPHABET 2       /* a stream alphabet exceeded L */
#define LQ_ST_TIE_UNPINNED 4   /* reserved, never raised: tables follow numpy's argsort order at every size */

/* dtype codes for activations */
#define LQ_F16 0
#define LQ_BF16 1
#define LQ_F32 2

/* Device table of one rANS stream (chunk tables and generic tables).
 * enc[s] = freq | cum << 11 | nb << 21 where nb = 11 - bitlen(freq). */
typedef struct {
    int32_t lo;          /* alphabet[0]; the alphabet is lo .. lo + n_sym - 1 */
    int32_t n_sym;       /* 0 when the stream is absent (its coset is empty) */
    int32_t n_symbols;   /* number of symbols in the stream */
    int32_t status;
    uint32_t enc[LQ_MAXSYM];
} lq_table;

int lq_version(void);
const char *lq_status_string(int code);
/* HIP runtime version this library is running against (hipRuntimeGetVersion). */
int lq_hip_runtime_version(void);

/* ---------------------------------------------------------------- E8 ---- */

/* encode_e8 / encode_d8 on fp32 (n, 8).  mode 0: E8, 1: D8.
 * Replaces core/e8_quantizer.py:20-83 (encode_d8, encode_e8). */
int lq_e8_encode_f32(const float *d_x, int64_t n, int mode, float *d_out, hipStream_t s);

/* e8_to_symbols on fp32 E8 points: coset (n) and 8 int32 symbols per vector
 * (7 free coordinates + floor(c7/2)).  Replaces core/entropy_coder.py:46-68. */
int lq_e8_to_symbols(const float *d_q, int64_t n, int32_t *d_coset, int32_t *d_sym8, hipStream_t s);

/* symbols_to_e8.  Replaces core/entropy_coder.py:71-89. */
int lq_symbols_to_e8(const int32_t *d_coset, const int32_t *d_sym8, int64_t n, float *d_q, hipStream_t s);

/* Per-head sigma^2 = mean(x^2), fp32 scale sqrt(2*pi*e*sigma^2*4^-b) (1 if
 * sigma^2 < 1e-12) and its fp16 copy; bits per chunk.  Also the per-head
 * fast-division word consumed by lq_chunk_quantize: 0 (IEEE division), or,
 * when x * r corrected by one FMA equals x / scale for every fp16 input, the
 * fp32 bit pattern of r = RN(1 / scale) (never 0; consumers test != 0 and
 * take r from it).  d_work: 4096 + n_heads_total doubles.
 * Replaces llm/compressed_kv_cache.py:188-196. */
int lq_head_scales(const void *d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                   const int32_t *d_chunk_bits, double *d_work, float *d_sigma2, float *d_scale32,
                   uint16_t *d_scale16, int32_t *d_fastdiv, hipStream_t s);

/* Rotated rows (the long-context path): as lq_head_scales on w = RHT(x), the
 * randomized Hadamard transform of each head_dim row (forward: FWHT(x * s) /
 * sqrt(head_dim) in fp32, sign row s = d_signs[head], head = chunk * n_heads + h,
 * d_signs (n_chunks * n_heads, head_dim) fp32 +-1), computed in registers:
 * no rotated copy is written.  head_dim a power of two in [8, 128], bph a
 * multiple of head_dim / 8.  d_fastdiv receives 0 (rotated values are fp32).
 * Replaces core/pipeline.py:100-108 (RHT.forward) + llm/perplexity_eval.py:35-61
 * (HeadRHT) feeding llm/compressed_kv_cache.py:188-196. */
int lq_head_scales_rht(const void *d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim,
                       const float *d_signs, const int32_t *d_chunk_bits, double *d_work, float *d_sigma2,
                       float *d_scale32, uint16_t *d_scale16, int32_t *d_fastdiv, hipStream_t s);

/* Fast-division words for caller-supplied fp32 scales (exhaustive check of all
 * 2048 fp16 significands per head).  Same d_fastdiv words as above. */
int lq_scale_fastdiv(const float *d_scale32, int64_t n_heads_total, int dtype, int32_t *d_fastdiv,
                     hipStream_t s);

/* Quantize a batch of chunks: x / scale -> E8 nearest point -> symbols.
 * Writes, per chunk: int8 symbols grouped per LQ_BLK block, coset-0 columns
 * then coset-1 columns, the 8 columns of a coset interleaved in 16-byte units
 * (d_sym, n_chunks * nblk * LQ_SYM_STRIDE bytes), the coset
 * bitmap in the reference's LSB-first byte order (d_coset_bits,
 * n_chunks * nblk * LQ_BLK / 8 bytes), the coset-1 count per block (d_blk_n1),
 * the 16 x 256 symbol histograms (d_hist, must be zero on entry) and status
 * bits.  d_deq (nullable) receives q * scale32 in deq_dtype, the value
 * update() returns.  d_dither_seed (nullable, one int64 per chunk) turns on the
 * subtractive dither of the rotated path: d in [-1, 1)^8 per vector from
 * SplitMix64 of (seed, vector index) is added to x / scale before the search
 * and removed in d_deq ((q - d) * scale32); no counterpart in the reference.
 * bph must not exceed 2^30 (LQ_ERR_ARG).
 * Replaces llm/compressed_kv_cache.py:199-231,270. */
int lq_chunk_quantize(const void *d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                      const float *d_scale32, const int32_t *d_fastdiv, int8_t *d_sym,
                      uint8_t *d_coset_bits, uint32_t *d_blk_n1, uint32_t *d_hist, int32_t *d_status,
                      void *d_deq, int deq_dtype, const int64_t *d_dither_seed, hipStream_t s);

/* Small updates without entropy coding (a decode step's K / V): the scales of
 * lq_head_scales and the dequantised rows q * scale32 of lq_chunk_quantize
 * (d_deq, x's dtype and layout) in one call.  d_work: scratch of
 * lq_quantize_deq_workspace(n_chunks, n_heads, bph) bytes (-1: invalid
 * geometry), 256-byte aligned, contents need not be cleared; calls sharing it
 * must be ordered on one stream.  Replaces llm/compressed_kv_cache.py:188-221
 * for the eval_only_no_entropy path and the quantize half of update(). */
int64_t lq_quantize_deq_workspace(int64_t n_chunks, int64_t n_heads, int64_t bph);
int lq_quantize_deq(const void *d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                    const int32_t *d_chunk_bits, void *d_work, float *d_sigma2, float *d_scale32,
                    uint16_t *d_scale16, void *d_deq, hipStream_t s);

/* Rotated rows: lq_chunk_quantize of w = RHT(x) (as lq_head_scales_rht), the
 * rotation in registers, the scale division rounded as IEEE division, optional dither; no
 * dequantised output.  Same outputs and layouts as lq_chunk_quantize on a
 * materialised fp32 rotation.  Replaces core/pipeline.py:100-108 +
 * llm/perplexity_eval.py:35-61 feeding llm/compressed_kv_cache.py:199-231,270. */
int lq_chunk_quantize_rht(const void *d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim,
                          const float *d_signs, const float *d_scale32, int8_t *d_sym, uint8_t *d_coset_bits,
                          uint32_t *d_blk_n1, uint32_t *d_hist, int32_t *d_status, const int64_t *d_dither_seed,
                          hipStream_t s);

/* Wide path (alphabets up to L = 1024 symbols, e.g. heavy-tailed K at low
 * rates): as lq_chunk_quantize with int16 symbols (n_chunks * nblk *
 * LQ_SYM_STRIDE int16) and, instead of histograms, per-stream min / max in
 * d_minmax (n_chunks * 16 * 2 int32, initialised to INT_MAX / INT_MIN).  A
 * symbol outside int16 sets LQ_ST_SYM_OVERFLOW.  Followed by
 * lq_chunk_hist_wide, lq_chunk_tables_wide, lq_chunk_encode_wide and the
 * shared lq_chunk_pack / lq_chunk_decode.  Replaces the same reference lines
 * as lq_chunk_quantize (llm/compressed_kv_cache.py:199-231,270). */
int lq_chunk_quantize_wide(const void *d_x, int dtype, int64_t n_chunks, int64_t n_heads, int64_t bph,
                           const float *d_scale32, const int32_t *d_fastdiv, int16_t *d_sym, uint8_t *d_coset_bits,
                           uint32_t *d_blk_n1, int32_t *d_minmax, int32_t *d_status, void *d_deq, int deq_dtype,
                           const int64_t *d_dither_seed, hipStream_t s);

/* Coarse / fine escape of the wide path, for streams whose alphabet exceeds
 * L = 1024 symbols (the reference's table normalisation, core/gpu_ans.py:73-84,
 * never terminates there; this format is defined by this build and has no
 * reference counterpart).  Plan: per chunk and coordinate j, the least
 * k_j in [0, 7] with (max >> k_j) - (min >> k_j) + 5 <= L for both cosets'
 * streams of j (d_esc_k: n_chunks * 8 int32), and the coarse min / max of
 * every stream (d_minmax_coarse, layout of d_minmax), which then feed
 * lq_chunk_hist_wide and lq_chunk_tables_wide.  No k fits: LQ_ST_ALPHABET. */
int lq_chunk_escape_plan(const int32_t *d_minmax, int64_t n_chunks, int32_t *d_esc_k, int32_t *d_minmax_coarse,
                         int32_t *d_status, hipStream_t s);

/* Escape split: in the int16 staging of lq_chunk_quantize_wide, every symbol
 * s of a coordinate with k_j > 0 becomes s >> k_j (floor), and its k_j low
 * bits go to d_fine: coordinate j of chunk c owns nblk * 16 * k_j words from
 * word d_fine_off[c * 8 + j], vector v's bits at bit v * k_j, least
 * significant first.  Chunks with every k_j = 0 are left untouched. */
int lq_chunk_escape_split(int16_t *d_sym, const uint8_t *d_coset_bits, const uint32_t *d_blk_n1, int64_t n_chunks,
                          int64_t n_vectors, const int32_t *d_esc_k, const int64_t *d_fine_off, uint32_t *d_fine,
                          hipStream_t s);

/* Wide path: per-stream histograms (n_chunks * 16 * 1024 uint32, zero on
 * entry) of the int16 symbols in the window [min, min + 1023].
 * Replaces the np.unique counting of llm/compressed_kv_cache.py:242-246. */
int lq_chunk_hist_wide(const int16_t *d_sym, const uint32_t *d_blk_n1, int64_t n_chunks, int64_t n_vectors,
                       const int32_t *d_minmax, uint32_t *d_hist, hipStream_t s);

/* x / scale32[head] -> nearest E8 point (fp32 (n_heads * bph, 8)), head = vector / bph,
 * with the same arithmetic as lq_chunk_quantize.  d_fastdiv from lq_head_scales /
 * lq_scale_fastdiv.  Replaces llm/compressed_kv_cache.py:199-201 (x_scaled, encode_e8). */
int lq_e8_quantize_heads(const void *d_x, int dtype, int64_t n_heads, int64_t bph, const float *d_scale32,
                         const int32_t *d_fastdiv, float *d_q, hipStream_t s);

/* ------------------------------------------------------------------ rANS -- */

/* Chunk tables from the histograms: alphabet range(min-2, max+2) and
 * build_rans_table normalisation with numpy's argsort tie order.
 * Replaces llm/compressed_kv_cache.py:242-250 + core/gpu_ans.py:62-98. */
int lq_chunk_tables(const uint32_t *d_hist, int64_t n_chunks, lq_table *d_tables, int32_t *d_status,
                    hipStream_t s);

/* Wide-path tables: alphabet range(min-2, max+2) from d_minmax, counts from
 * lq_chunk_hist_wide; an alphabet above L = 1024 symbols (where the
 * reference's normalisation loop never ends) sets LQ_ST_ALPHABET in the
 * table and the chunk status and leaves the stream empty.
 * Replaces llm/compressed_kv_cache.py:242-250 + core/gpu_ans.py:62-98. */
int lq_chunk_tables_wide(const uint32_t *d_hist, const int32_t *d_minmax, int64_t n_chunks, lq_table *d_tables,
                         int32_t *d_status, hipStream_t s);

/* Workspace of the chunk encoder, in bytes. */
int64_t lq_chunk_encode_workspace(int64_t n_chunks, int64_t n_vectors);

/* Encode every stream of a batch of chunks (one lane per block and stream).
 * Outputs per (chunk, stream, block): bit offset in the stream (d_blk_off) and
 * decoder checkpoint state (d_blk_state); per (chunk, stream): n_bits,
 * final state and word offset inside the chunk bitstream; per chunk: total
 * words (d_chunk_words).  Words are written by lq_chunk_pack.
 * Replaces llm/compressed_kv_cache.py:236-263 + core/gpu_ans.py:105-139. */
int lq_chunk_encode(const int8_t *d_sym, const uint32_t *d_blk_n1, int64_t n_chunks, int64_t n_vectors,
                    const lq_table *d_tables, void *d_work, uint32_t *d_blk_off, uint16_t *d_blk_state,
                    int64_t *d_stream_nbits, int32_t *d_stream_state, int64_t *d_stream_woff,
                    int64_t *d_chunk_words, hipStream_t s);

/* lq_chunk_encode on the wide path's int16 symbols (same outputs). */
int lq_chunk_encode_wide(const int16_t *d_sym, const uint32_t *d_blk_n1, int64_t n_chunks, int64_t n_vectors,
                         const lq_table *d_tables, void *d_work, uint32_t *d_blk_off, uint16_t *d_blk_state,
                         int64_t *d_stream_nbits, int32_t *d_stream_state, int64_t *d_stream_woff,
                         int64_t *d_chunk_words, hipStream_t s);

/* Write the merged bitstreams: chunk c's words start at d_words + d_chunk_base[c]
 * (caller-chosen, e.g. an exclusive prefix of d_chunk_words).  Each stream is
 * the reference's layout: LSB-first bits, n_words + 1 words, last word zero. */
int lq_chunk_pack(int64_t n_chunks, int64_t n_vectors, const lq_table *d_tables, const void *d_work,
                  const uint32_t *d_blk_off, const int64_t *d_stream_nbits, const int64_t *d_stream_woff,
                  const int64_t *d_chunk_base, uint32_t *d_words, hipStream_t s);

/* Decode + dequantize a batch of chunks to (B, H, T, hd) in out_dtype:
 * fp16(q * float(scale16[head])).  d_lut_work: n_chunks * 16 * 1024 uint32.
 * d_words must have 2 readable words after the last chunk's last stream.
 * d_dither_seed (nullable): the seeds the chunks were quantized with; the
 * output is then (q - d) * scale16 (fp32 arithmetic, then out_dtype).
 * Replaces llm/compressed_kv_cache.py:289-332 (_decompress_chunk). */
int lq_chunk_decode(const uint32_t *d_words, const int64_t *d_chunk_base, const int64_t *d_stream_woff,
                    const uint32_t *d_blk_off, const int64_t *d_stream_nbits, const uint16_t *d_blk_state, const uint8_t *d_coset_bits,
                    const uint32_t *d_blk_n1, const lq_table *d_tables, const uint16_t *d_scale16,
                    int64_t n_chunks, int64_t n_heads, int64_t bph, uint32_t *d_lut_work, void *d_out,
                    int out_dtype, const int64_t *d_dither_seed, hipStream_t s);

/* lq_chunk_decode (d_signs null) or lq_chunk_decode_rht (d_signs given) of a
 * batch with escaped chunks (lq_chunk_escape_plan / lq_chunk_escape_split):
 * symbol j of a vector is (decoded coarse symbol << k_j) plus its low bits
 * from d_fine before c7 and the coset offset are applied.  Build-defined
 * format: no reference counterpart (the reference never terminates on such
 * streams). */
int lq_chunk_decode_escaped(const uint32_t *d_words, const int64_t *d_chunk_base, const int64_t *d_stream_woff,
                            const uint32_t *d_blk_off, const int64_t *d_stream_nbits, const uint16_t *d_blk_state,
                            const uint8_t *d_coset_bits, const lq_table *d_tables, const uint16_t *d_scale16,
                            int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim, const float *d_signs,
                            const int32_t *d_esc_k, const int64_t *d_fine_off, const uint32_t *d_fine,
                            uint32_t *d_lut_work, void *d_out, int out_dtype, const int64_t *d_dither_seed, hipStream_t s);

/* lq_chunk_decode of chunks written by lq_chunk_quantize_rht: each row's
 * fp32 dequantised values ((q - d) * scale16) are rotated back (FWHT / sqrt(head_dim),
 * then * s, d_signs as for lq_chunk_quantize_rht) before the out_dtype store;
 * head_dim a power of two in [8, 128].  Replaces llm/compressed_kv_cache.py:289-332
 * followed by core/pipeline.py:110-118 (RHT.inverse). */
int lq_chunk_decode_rht(const uint32_t *d_words, const int64_t *d_chunk_base, const int64_t *d_stream_woff,
                        const uint32_t *d_blk_off, const int64_t *d_stream_nbits, const uint16_t *d_blk_state,
                        const uint8_t *d_coset_bits, const lq_table *d_tables, const uint16_t *d_scale16,
                        int64_t n_chunks, int64_t n_heads, int64_t bph, int head_dim, const float *d_signs,
                        uint32_t *d_lut_work, void *d_out, int out_dtype, const int64_t *d_dither_seed, hipStream_t s);

/* Decoder LUTs of every stream of a chunk batch (n_chunks * 16 * 1024 uint32:
 * per slot: 31 - k | k << 5 | symbol index << 9 | (row * 1024 + (x' << k) - 1024) << 19,
 * with x' = freq + slot - cum, k its renormalisation bits and row = stream & 7),
 * as lq_chunk_decode builds them internally.  Part of the table stage of core/gpu_ans.py:88-95 (lookup). */
int lq_chunk_luts(const lq_table *d_tables, int64_t n_chunks, uint32_t *d_lut, hipStream_t s);

/* ---------------------------------------------------- decode attention --- */

/* Device pointers of a batch of chunks in lq_chunk_encode's format (one
 * EncodedBatch of the host side), with the per-chunk geometry. */
typedef struct {
    const uint32_t *words;
    const int64_t *chunk_base;
    const int64_t *stream_woff;
    const uint32_t *blk_off;
    const int64_t *stream_nbits;
    const uint16_t *blk_state;
    const uint8_t *coset_bits;
    const uint32_t *blk_n1;
    const lq_table *tables;
    const uint16_t *scale16;
    int64_t n_chunks;
    int64_t n_heads;   /* B * H_kv */
    int64_t bph;       /* T * hd / 8 vectors per head */
} lq_chunk_batch;

/* Workspace of lq_decode_attention, in bytes. */
int64_t lq_attn_workspace(int64_t n_chunks, int64_t n_heads, int64_t bph, int group);

/* One decode step of attention over a compressed prefix + fp16 tail:
 * out[qh] = softmax(q[qh] . K^T / sqrt(128)) V for every query head qh, with
 * kv head qh / group.  K, V: chunk batches of the same geometry (head_dim 128,
 * tokens per chunk a multiple of 32), dequantised as _decompress_chunk does
 * (lattice point times the fp16-stored scale); chunk c holds tokens
 * c*T .. c*T+T-1 of the prefix.  Tail: (n_heads, t_tail, 128) fp16 K and V,
 * t_tail <= 1024, following the prefix.  q, out: (n_heads * group, 128) fp16.
 * Replaces the decompress -> torch.cat -> SDPA read of
 * llm/compressed_kv_cache.py:384-395 (and the fused merge of
 * llm/fused_triton_merge.py:33-130 feeding attention). */
int lq_decode_attention(const lq_chunk_batch *k, const lq_chunk_batch *v, const uint16_t *d_q, int group,
                        const uint16_t *d_tail_k, const uint16_t *d_tail_v, int64_t t_tail, void *d_work,
                        uint16_t *d_out, hipStream_t s);

/* Generic tables (build_rans_table API): n_tables histograms of n_sym[t] <= 1024
 * counts at d_counts + d_count_off[t].  Outputs freqs / cumfreqs (n_sym+1) at the
 * same offsets (+t for cum), lookup (1024 per table) and status per table.
 * Replaces core/gpu_ans.py:62-98. */
int lq_build_tables(const int64_t *d_counts, const int64_t *d_count_off, const int32_t *d_n_sym,
                    int32_t n_tables, int32_t *d_freqs, int32_t *d_cum, int32_t *d_lookup, int32_t *d_status,
                    hipStream_t s);

/* Serial rANS encode of n_streams streams of symbol indices (one lane each).
 * Stream t: d_idx + d_sym_off[t], length d_n[t], table freqs/cum at
 * d_tab_off[t].  Words go to d_words + d_word_off[t] (capacity
 * 10*n/32 + 2 words each); state and n_bits per stream.
 * d_scratch: same total capacity as d_words.  Replaces core/gpu_ans.py:105-139. */
int lq_rans_encode_streams(const int32_t *d_idx, const int64_t *d_sym_off, const int64_t *d_n,
                           const int32_t *d_freqs, const int32_t *d_cum, const int64_t *d_tab_off,
                           int32_t n_streams, uint32_t *d_scratch, uint32_t *d_words, const int64_t *d_word_off,
                           int64_t *d_state, int64_t *d_nbits, hipStream_t s);

/* One lane per stream decode with the reference's bit-position guard; writes
 * int64 symbol values.  Replaces _rans_decode_kernel (core/gpu_ans.py:175-235). */
int lq_rans_decode_streams(const int32_t *d_bits, const int32_t *d_bit_off, const int32_t *d_nbits,
                           const int32_t *d_init, const int32_t *d_ndec, const int32_t *d_lookup,
                           const int32_t *d_freqs, const int32_t *d_cum, const int32_t *d_alphabet,
                           const int32_t *d_tid, int32_t max_sym, const int32_t *d_out_off, int32_t n_streams,
                           int64_t *d_out, hipStream_t s);

/* -------------------------------------------------------- compact form --- */

/* Fixed-rate unpack + dequant, b in {3,4,5}: out = fp16((coord + 0.5*coset) * scale[head_idx]).
 * d_scales holds n_scales values; a head index outside [0, n_scales) is clamped
 * (garbage out, no fault, no host check).
 * Replaces _unpack_e8_4bit_kernel (core/triton_dequant.py:45-132). */
int lq_unpack_compact(const uint8_t *d_packed, int bits, int64_t n, const float *d_scales, int64_t n_scales,
                      const int32_t *d_head_idx, uint16_t *d_out, hipStream_t s);

/* Fixed-rate pack of in-range E8 points, b in {3,4,5} (core/compact_storage.py:87-154).
 * d_ok (n) receives 1 for a valid in-range point; invalid points are written as zero bytes. */
int lq_pack_compact(const float *d_q, int bits, int64_t n, uint8_t *d_packed, int32_t *d_ok, hipStream_t s);

/* Single-pass repr/fallback merge: block i is decoded from packed[rank_repr(i)]
 * when mask[i] != 0 else copied from fallback[rank_fb(i)]; ranks are computed
 * in-kernel (wave ballots within 1024-block tiles, a chained look-back across
 * them; the workspace is cleared by the call).  head = i / bph.  Replaces _fused_merge_4bit_vec_kernel
 * (llm/fused_triton_merge.py:33-130), with unpack_e8's floor-mod parity.
 * packed holds n_packed rows, fallback n_fallback; ranks past them (a mask
 * that selects more rows than the caller holds) are clamped, and a block with
 * no row at all is written as zeros: garbage out, no fault, no host check.
 * d_work: lq_merge_workspace(total) bytes.  After the call the int32 at byte
 * offset (tiles + 1) * 8 of d_work (tiles = ceil(total / 1024)) is nonzero if
 * a tile's look-back wait did not end; d_out is then invalid. */
int64_t lq_merge_workspace(int64_t total_blocks);
int lq_fused_merge(const uint8_t *d_packed, int64_t n_packed, int bits, const uint16_t *d_fallback,
                   int64_t n_fallback, const uint8_t *d_mask, const float *d_scales, int64_t total_blocks,
                   int64_t bph, void *d_work, uint16_t *d_out, hipStream_t s);

/* Fixed-rate compression of a (n_heads, bph) batch in one pass: x / scale32[head]
 * (three-op division where d_fastdiv says so, as lq_chunk_quantize) -> nearest
 * E8 point; a point in range at `bits` goes to d_packed (b bytes, the
 * pack_e8 layout) at its rank among the in-range points, any other to
 * d_fallback as fp16(q * float(scale16[head])) at its rank among the rest;
 * d_mask gets 1 / 0 per vector, d_repr_heads (nullable) the head of each
 * packed point in packed order, d_tile_off the number of in-range points
 * before each 1024-vector tile (what lq_compact_merge takes) and d_totals
 * (3 int64: n_packed, n_fallback, error word).  d_packed / d_fallback hold
 * room for every vector (n * b and n * 16 bytes); only the first d_totals rows
 * are written.  No host sync.  The error word is cleared by the call and set
 * when a tile's look-back wait does not end; every output is then invalid, so
 * a caller reads it with the counts (one copy) and discards the batch.
 * d_work: lq_compact_encode_workspace(n) bytes (cleared by the call).
 * Replaces core/compact_storage.py:338-357 (quantize_and_pack) with the fp16
 * fallback of the fixed-rate cache (llm/fused_triton_merge.py chunk fields). */
int64_t lq_compact_encode_workspace(int64_t n);
int lq_compact_encode(const void *d_x, int dtype, int64_t n_heads, int64_t bph, const float *d_scale32,
                      const int32_t *d_fastdiv, const uint16_t *d_scale16, int bits, uint8_t *d_mask,
                      uint8_t *d_packed, uint16_t *d_fallback, int32_t *d_repr_heads, int64_t *d_tile_off,
                      int64_t *d_totals, void *d_work, hipStream_t s);

/* lq_compact_encode with the per-head scales computed on the way (two
 * launches in all): sigma^2 as lq_head_scales forms it (same partial sums,
 * same order, so bit-identical), scale = sqrt(f32(2 pi e) sigma^2 4^-scale_bits)
 * (1 where sigma^2 < 1e-12), its fp16 copy, float(scale16) for the merge, and
 * the fast-division flags, all finalised inside the encoder, whose tiles of
 * 1024 vectors then span at most two heads: bph >= 1024 is required
 * (LQ_ERR_ARG otherwise; lq_head_scales + lq_compact_encode serve the rest).
 * d_sigma2 may be NULL.  d_work: lq_compact_encode_scaled_workspace bytes,
 * cleared by the call.  Outputs, totals and error word as lq_compact_encode.
 * Replaces llm/compressed_kv_cache.py:188-196 (scales) with
 * core/compact_storage.py:338-357 as lq_compact_encode does. */
int64_t lq_compact_encode_scaled_workspace(int64_t n_heads, int64_t bph);
int lq_compact_encode_scaled(const void *d_x, int dtype, int64_t n_heads, int64_t bph, int scale_bits, int bits,
                             float *d_sigma2, float *d_scale32, uint16_t *d_scale16, float *d_scale16f,
                             uint8_t *d_mask, uint8_t *d_packed, uint16_t *d_fallback, int32_t *d_repr_heads,
                             int64_t *d_tile_off, int64_t *d_totals, void *d_work, hipStream_t s);

/* lq_fused_merge with the tile offsets lq_compact_encode wrote (no count or
 * scan pass).  Replaces llm/fused_triton_merge.py:33-172 as lq_fused_merge. */
int lq_compact_merge(const uint8_t *d_packed, int64_t n_packed, int bits, const uint16_t *d_fallback,
                     int64_t n_fallback, const uint8_t *d_mask, const float *d_scales, int64_t total_blocks,
                     int64_t bph, const int64_t *d_tile_off, uint16_t *d_out, hipStream_t s);

/* ----------------------------------------------------------- API helpers -- */

/* validate_e8 + check_representable on fp32 points (n, 8): per point
 * LQ_V_VALID (consistently integer or half-integer, even integer sum, within
 * atol), LQ_V_HALF (the half-integer coset) and, for bits in {3,4,5},
 * LQ_V_INRANGE (valid and every integer coordinate in [-2^(b-1), 2^(b-1)-1]).
 * Replaces core/compact_storage.py:39-80 (validate_e8), :235-249 (check_representable). */
#define LQ_V_VALID 1
#define LQ_V_HALF 2
#define LQ_V_INRANGE 4
int lq_e8_validate(const float *d_q, int64_t n, float atol, int bits, int32_t *d_flags, hipStream_t s);

/* unpack_e8 to fp32 lattice points (n, 8), b in {3,4,5}, big-endian b-byte words.
 * Replaces core/compact_storage.py:157-222. */
int lq_unpack_e8(const uint8_t *d_packed, int bits, int64_t n, float *d_q, hipStream_t s);

/* Symbol values -> table indices with rans_encode's rule: an equal alphabet
 * entry (the last one), else the first entry at minimal distance.
 * contiguous != 0 declares alphabet = lo, lo+1, ..  (n_alphabet <= 1024).
 * Replaces the lookup in core/gpu_ans.py:110-119. */
int lq_symbol_index(const int64_t *d_sym, int64_t n, const int64_t *d_alphabet, int32_t n_alphabet, int contiguous,
                    int32_t *d_idx, hipStream_t s);

/* Coset bit packing, LSB-first: bit i -> byte i/8, bit i%8 (d_coset: uint8 0/1).
 * Replaces llm/compressed_kv_cache.py:46-54 and :57-63. */
int lq_pack_coset_bits(const uint8_t *d_coset, int64_t n, uint8_t *d_out, hipStream_t s);
int lq_unpack_coset_bits(const uint8_t *d_packed, int64_t n, uint8_t *d_out, hipStream_t s);

/* Randomized Hadamard transform of n_rows rows of d (power of two, 8..512)
 * elements: forward FWHT(x * signs) / sqrt(d), inverse FWHT(x) / sqrt(d) * signs,
 * fp32 arithmetic in the reference's butterfly order.  Row r uses sign row
 * (r / rows_per_sign) % n_sign of d_signs (n_sign, d) fp32.
 * Replaces core/pipeline.py:49-118 (fast_hadamard_transform, RHT) and
 * llm/perplexity_eval.py:35-61 (HeadRHT). */
int lq_rht(const void *d_x, int in_dtype, int64_t n_rows, int d, const float *d_signs, int64_t rows_per_sign,
           int n_sign, int inverse, void *d_out, int out_dtype, hipStream_t s);

/* ------------------------------------------------------ resident form --- */

/* Fixed-width resident form of a compressed KV prefix (head_dim 128), read by
 * lq_resident_attention.  Per kv head, tokens in blocks of 16; per block 256
 * vector records laid out [group 0..3][slot 0..63] (record (slot, group) is
 * vector 4*group + slot/16 of token 16*block + slot%16).  A record is the
 * reference's b = 5 fixed-rate code word of the lattice point
 * (core/compact_storage.py:87-154: coset, c0..c6 + 16 in 5 bits, (c7 + 16) >> 1
 * in 4 bits, c7's low bit = parity of c0..c6), its 40 bits split as
 *   a (uint32): coset @0, u0 @1, u2 @6, u4 @11, bit 3 of c7h @16, u1 @17, u3 @22, u5 @27
 *   b (uint8):  u6 @0, bits 0..2 of c7h @5
 * (u_i = c_i + 16, c7h = u7 >> 1).  Vectors with a coordinate outside [-16, 15]
 * are exceptions (bit slot of mask[block][group]); their lattice point is kept
 * as 8 int16 values 2c in exc[], block entries from meta[block].base on, in
 * (group, slot) order -- the representable-or-fallback split of
 * llm/fused_triton_merge.py:33-130 with lattice values as the fallback.
 * meta[block] = {header low, header high, base, count}: the 64-bit header
 * repeats the first seven exceptions for the attention kernel (byte 0 = count
 * saturated at 255, byte 1 + k = slot | group << 6 of exception k), base is
 * the index of the block's first entry in exc[].  scale[token] is the fp16
 * scale the token's chunk stores. */
typedef struct {
    uint32_t *a;             /* [n_heads][cap_blocks][4][64] */
    uint8_t *b;              /* [n_heads][cap_blocks][4][64] */
    uint64_t *mask;          /* [n_heads][cap_blocks][4] */
    uint32_t *meta;          /* [n_heads][cap_blocks][4] */
    int16_t *exc;            /* [exc_cap][8] */
    uint16_t *scale;         /* [n_heads][cap_blocks * 16] fp16 */
    int32_t *n_exc;          /* device counter: exception entries in use */
    int32_t *status;         /* device flags: LQ_RES_ST_* */
    int64_t n_heads;
    int64_t cap_blocks;
    int64_t exc_cap;
} lq_resident;

#define LQ_RES_ST_EXC_OVERFLOW 1  /* more exceptions than exc_cap: entries beyond it were dropped */

/* Workspace (bytes) of lq_resident_quantize for n_heads x t_tokens. */
int64_t lq_resident_workspace(int64_t n_heads, int64_t t_tokens);

/* Quantize x (n_heads, t_tokens, 128) of dtype into blocks blk0 .. blk0 + t_tokens/16
 * of resident heads h0 .. h0 + n_heads (t_tokens a multiple of 16): the lattice
 * point of every vector is encode_e8(x / scale32[head]) (core/e8_quantizer.py:61-83,
 * the division and decisions of llm/compressed_kv_cache.py:197-201), so it is the
 * point the chunk codec codes with the same scales; scale16[head] is stored per
 * token.  Exception entries are appended at *n_exc (capacity exc_cap; overflow
 * sets LQ_RES_ST_EXC_OVERFLOW).  Stream-ordered, no host sync. */
int lq_resident_quantize(const void *d_x, int dtype, int64_t n_heads, int64_t t_tokens, const float *d_scale32,
                         const uint16_t *d_scale16, const lq_resident *r, int64_t h0, int64_t blk0, void *d_work,
                         hipStream_t s);

/* Dequantise resident blocks back to (n_heads, n_blocks*16, 128) fp16 / bf16 / fp32:
 * lattice point times the stored fp16 scale, rounded once, as _decompress_chunk
 * writes it (llm/compressed_kv_cache.py:289-332). */
int lq_resident_dequant(const lq_resident *r, int64_t h0, int64_t n_heads, int64_t blk0, int64_t n_blocks,
                        void *d_out, int out_dtype, hipStream_t s);

/* Workspace (bytes) of lq_resident_attention; its first n_heads uint32 are
 * completion counters that must be zero before the first call (each call leaves
 * them zero). */
int64_t lq_resident_attn_workspace(int64_t n_heads, int group, int64_t t_prefix, int64_t t_tail);

/* One decode step of attention over resident prefixes + fp16 tail:
 * out[qh] = softmax(q[qh] . K^T / sqrt(128)) V, kv head qh / group, over the
 * first t_prefix tokens (a multiple of 16) of resident heads 0 .. n_heads of k
 * and v, then t_tail tokens of tail_k / tail_v (n_heads, t_tail, 128) fp16.
 * q, out: (n_heads * group, 128) fp16; group 1..16.  Replaces the fp16-resident
 * read of llm/compressed_kv_cache.py:384-395 + HF attention, and the fused
 * merge of llm/fused_triton_merge.py:33-130 that joins packed vectors with
 * their fallback before attention. */
int lq_resident_attention(const lq_resident *k, const lq_resident *v, int64_t t_prefix, const uint16_t *d_q,
                          int group, const uint16_t *d_tail_k, const uint16_t *d_tail_v, int64_t t_tail,
                          void *d_work, uint16_t *d_out, hipStream_t s);

/* Bytes of the device scratch array behind lq_resident_attention_noalloc. */
#define LQ_RES_ATTN_SCRATCH_BYTES (4 << 20)

/* lq_resident_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  No counterpart in the reference.  The counters and split
 * records live in a file-scope device array of LQ_RES_ATTN_SCRATCH_BYTES per
 * device, held until the process ends; its address is looked up (and its
 * counter region cleared by a fill kernel) on the first call on each device,
 * with that device current: make that first call outside stream capture.  The
 * array holds completion counters for up to 1024 kv heads at a fixed place
 * (each completed call leaves them zero) and then the split records: a step
 * with more kv heads, or whose records exceed the rest of the array, returns
 * LQ_ERR_SCRATCH without launching.  Nothing is allocated: no hipMalloc or
 * hipFree.  Calls on one device share the array, so calls that overlap on one
 * GPU (different streams, or different host threads) race; calls in stream
 * order do not.  Results equal lq_resident_attention's within 2 fp16 ulps
 * (prefix tiles are dealt to waves dynamically, so the summation order of a
 * head's partial results can differ between calls). */
int lq_resident_attention_noalloc(const lq_resident *k, const lq_resident *v, int64_t t_prefix, const uint16_t *d_q,
                                  int group, const uint16_t *d_tail_k, const uint16_t *d_tail_v, int64_t t_tail,
                                  uint16_t *d_out, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif /* LATTICEQUANT_AMD_H */

/*
 * bitcache C ABI: compressed KV-cache decode attention for AMD Instinct MI355X (gfx950).
 *
 * Plain C: raw device pointers, integer sizes, a HIP stream handle passed as
 * void*, and an int status (0 = ok).  No entry point allocates device memory,
 * synchronises the device or aborts the process.  Work is enqueued
 * asynchronously on `stream` (NULL = the legacy default stream).
 *
 * Blob format ("dense planar", opaque to callers).  A binary blob of capacity
 * n vectors is n * bc_sizeof_binary_vec() = n * 36 bytes, a residual blob is
 * n * bc_sizeof_residual_vec() = n * 130 bytes -- the same sizes the
 * reference's BinaryVec / ResidualVec arrays occupy -- but the bytes are laid
 * out for streaming:
 *   binary blob   [0, n*d/8)        sign bits of vector v at v*d/8, bit i of the
 *                                   vector = bit i%8 of byte i/8 (identical to the
 *                                   reference's little-endian uint32 words)
 *                 [n*d/8, +2n)      fp16 mean-|x| scale of vector v at n*d/8 + 2v
 *   residual blob [0, n*d/2)        INT4 codes of vector v at v*d/2, element 2j in
 *                                   the low nibble of byte j (as the reference)
 *                 [n*d/2, +2n)      fp16 residual absmax of vector v at n*d/2 + 2v
 * The bytes past these planes (up to n*36 and n*130) are unused: no encoder
 * writes them and no kernel reads them, so their content is whatever the
 * caller's allocation held.
 * The capacity n of a blob is implied by each entry point (documented per
 * function).  bc_binary_to_reference()/..._from_reference() convert to and from
 * the reference's array-of-structs bytes.
 *
 * Head dims: multiples of 32 up to 256 (the reference's MAX_HEAD_DIM).
 * Vectors are fp16.  Attention inputs: Q [batch, n_heads, head_dim]; cache
 * vector index = (b * n_kv_heads + kv_head) * kv_stride + position;
 * query head h reads kv head h / (n_heads / n_kv_heads).
 */
#ifndef BITCACHE_H_
#define BITCACHE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum bc_status {
    BC_OK = 0,
    BC_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative or inconsistent sizes */
    BC_ERR_UNSUPPORTED = 2,      /* head_dim not a multiple of 32 or above 256 */
    BC_ERR_WORKSPACE = 3,        /* workspace missing or smaller than required */
    BC_ERR_HIP = 4               /* the HIP runtime reported an error */
};

/* ---- library ------------------------------------------------------------ */
int bc_abi_version(void);
const char* bc_status_string(int status);
/* Message of the last failing call on the calling thread ("" if none). */
const char* bc_last_error(void);

/* sizeof(BinaryVec) / sizeof(ResidualVec) of the reference: 36 and 130.
 * Replaces src/torch_binding.cpp:165-166 (sizeof_binary_vec / sizeof_residual_vec). */
int64_t bc_sizeof_binary_vec(void);
int64_t bc_sizeof_residual_vec(void);

/* ---- encode --------------------------------------------------------------- */
/* Sign bits + fp16 mean-|x| scale of n_vecs fp16 vectors [n_vecs, head_dim].
 * Blob capacity = n_vecs.  Bit-exact with the reference, including the fp32
 * summation order of the scale.
 * Replaces launch_binary_encode (src/binary_encode.cu:62-80). */
int bc_binary_encode(const void* src, void* binary_blob, int64_t n_vecs, int head_dim,
                     void* stream);

/* INT4 residual of src against an existing binary blob (its bits and its
 * fp16-rounded scale).  Capacity of both blobs = n_vecs.
 * Replaces launch_residual_encode (src/residual.cu:80-98). */
int bc_residual_encode(const void* src, const void* binary_blob, void* residual_blob,
                       int64_t n_vecs, int head_dim, void* stream);

/* Both blobs in one pass over src (prefill).  scale_mode 0: identical bytes to
 * bc_binary_encode followed by bc_residual_encode; scale_mode 1: the residual is
 * taken against the fp32 mean, as bc_online_encode_token does.
 * residual_blob may be NULL (binary only).  Capacity of both blobs = n_vecs.
 * No counterpart in the reference (it needs two launches, src/binary_encode.cu:62,
 * src/residual.cu:80). */
int bc_encode_fused(const void* src, void* binary_blob, void* residual_blob, int64_t n_vecs,
                    int head_dim, int scale_mode, void* stream);

/* Encode one token per (b, head) [batch, n_heads, head_dim] into ring slot
 * current_len % max_seq of caches with capacity batch*n_heads*max_seq.
 * residual_cache may be NULL (binary-only cache: nothing is written there).
 * Replaces launch_online_encode_token (src/online_encode.cu:122-149). */
int bc_online_encode_token(const void* kv, void* binary_cache, void* residual_cache, int batch,
                           int n_heads, int head_dim, int64_t current_len, int max_seq,
                           void* stream);

/* Bulk prefill into ring caches: src [rows, seq, head_dim] (rows = batch*n_heads)
 * lands in slots start_pos .. start_pos+seq-1 of caches with capacity
 * rows*max_seq; scale_mode as bc_encode_fused (1 = the online-encode math).
 * residual_cache may be NULL.  No counterpart in the reference (which appends
 * one token per call, bitcache/__init__.py:95-113). */
int bc_encode_into_cache(const void* src, void* binary_cache, void* residual_cache, int64_t rows,
                         int seq, int head_dim, int start_pos, int max_seq, int scale_mode,
                         void* stream);

/* bc_encode_into_cache for a source in the [batch, seq, n_heads, head_dim]
 * layout many model stacks hold K/V in: vector (b, s, h) lands in slot
 * start_pos + s of row b*n_heads + h (caches of capacity batch*n_heads*max_seq),
 * with the same bytes as bc_encode_into_cache of the [batch, n_heads, seq,
 * head_dim] transpose.  No counterpart in the reference. */
int bc_encode_into_cache_bshd(const void* src, void* binary_cache, void* residual_cache, int batch,
                              int seq, int n_heads, int head_dim, int start_pos, int max_seq,
                              int scale_mode, void* stream);

/* K and V of one decode step in a single launch (same semantics as two
 * bc_online_encode_token calls).  k_res / v_res may be NULL. */
int bc_online_encode_kv(const void* k, const void* v, void* k_bin, void* k_res, void* v_bin,
                        void* v_res, int batch, int n_heads, int head_dim, int64_t current_len,
                        int max_seq, void* stream);

/* Memory floor of bc_encode_fused: the same kernel, grid, loads and stores
 * with the arithmetic left out, so its time is what the access pattern alone
 * costs.  Writes meaningless bytes into both blobs (capacity n_vecs each).
 * head_dim 64, 128 or 256.  No counterpart in the reference; a measurement
 * aid for benchmarks. */
int bc_encode_traffic_probe(const void* src, void* binary_blob, void* residual_blob,
                            int64_t n_vecs, int head_dim, void* stream);

/* The device's streaming-read ceiling: reads n_bytes (a multiple of 16, src
 * 16-byte aligned) once with the nontemporal 16-byte loads the attention
 * kernels use for whole-KiB runs, spread over four workgroups per CU, and
 * writes one XOR word per wave into out (room for BC_READ_PROBE_OUT_WORDS
 * uint32).  Time it to read the attention kernels' bandwidth against what
 * the memory system delivers.  No counterpart in the reference; a
 * measurement aid for benchmarks. */
/* The device's mixed read/write ceiling for the encoders' traffic shape:
 * reads 3 * n_write_bytes from src (nontemporal 16-byte loads, three coalesced
 * KiB per wave) and writes n_write_bytes to dst (16 bytes per lane, whole
 * cache lines; nt_store != 0: nontemporal stores), four workgroups per CU.
 * n_write_bytes a multiple of 4096, src and dst 16-byte aligned.  No
 * counterpart in the reference; a measurement aid for benchmarks. */
int bc_mix_probe(const void* src, void* dst, int64_t n_write_bytes, int nt_store, void* stream);

#define BC_READ_PROBE_MAX_WGS 4096
#define BC_READ_PROBE_OUT_WORDS (4 * BC_READ_PROBE_MAX_WGS)
int bc_read_probe(const void* src, int64_t n_bytes, void* out, void* stream);

/* ---- attention -------------------------------------------------------------- */
/* Bytes of scratch the attention entry points need for this shape on the
 * current device (split-KV partial results).  Callers allocate it; it may be
 * reused across calls on the same stream. */
int bc_attention_workspace_size(int batch, int n_heads, int n_kv_heads, int seq_len,
                                int head_dim, size_t* bytes);

/* The key-split plan an attention call of this shape launches: n_splits per
 * (b, query-head group), the bytes of split partials it writes and the
 * workspace bc_attention_workspace_size reports (always >= partial_bytes).
 * (A plan of one split writes the output from its attention kernel; then
 * partial_bytes is what that split's partials would take.)
 * mode: BC_MODE_*; cu_count 0 plans for the current device, > 0 for a device
 * of that many CUs.  Allocates nothing and launches nothing.  No counterpart
 * in the reference; a diagnostic for callers sizing workspaces and for tests. */
#define BC_MODE_BINARY 0
#define BC_MODE_COMPENSATED 1
#define BC_MODE_ADAPTIVE 2
#define BC_MODE_HEAD_MODE 3
int bc_attention_split_plan(int mode, int batch, int n_heads, int n_kv_heads, int seq_len,
                            int head_dim, int cu_count, int* n_splits, size_t* partial_bytes,
                            size_t* workspace_bytes);

/* Binary-only decode attention, MHA, blob capacity batch*n_heads*seq_len.
 * Replaces launch_binary_attention (src/binary_attention.cu:84-105). */
int bc_binary_attention(const void* q, const void* k_bin, const void* v_bin, void* out, int batch,
                        int n_heads, int seq_len, int head_dim, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Residual-compensated decode attention, MHA, blob capacity batch*n_heads*seq_len.
 * Replaces launch_compensated_attention (src/compensated_attention.cu:111-134). */
int bc_compensated_attention(const void* q, const void* k_bin, const void* k_res,
                             const void* v_bin, const void* v_res, void* out, int batch,
                             int n_heads, int seq_len, int head_dim, void* workspace,
                             size_t workspace_bytes, void* stream);

/* General form: GQA (n_heads a multiple of n_kv_heads) and a ring-buffer
 * stride (blob capacity batch*n_kv_heads*kv_stride, keys [0, seq_len) valid).
 * k_res/v_res NULL selects binary attention.  No counterpart in the reference
 * (which assumes n_kv_heads == n_heads and kv_stride == seq_len). */
int bc_attention_gqa(const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                     const void* v_res, void* out, int batch, int n_heads, int n_kv_heads,
                     int seq_len, int kv_stride, int head_dim, void* workspace,
                     size_t workspace_bytes, void* stream);

/* bc_attention_gqa without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The split
 * partials live in a library-owned device array of 8 MiB per GPU (held until
 * the process ends); a shape whose partials need more returns
 * BC_ERR_WORKSPACE.  The call allocates nothing.  Calls that overlap on one
 * GPU (two streams, or two threads) share that array and race: serialise
 * them.  Same results as bc_attention_gqa. */
int bc_attention_gqa_noalloc(const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                             const void* v_res, void* out, int batch, int n_heads, int n_kv_heads,
                             int seq_len, int kv_stride, int head_dim, void* stream);

/* The two phases of bc_attention_gqa, for callers that schedule them
 * separately (e.g. merging partials of a sequence split across devices):
 * bc_attention_partial writes one (max, sum, acc[head_dim]) fp32 partial per
 * (b, query head, key split) into the workspace; bc_attention_combine merges
 * them into out.  Both take the shape arguments of bc_attention_gqa and the
 * same workspace.  No counterpart in the reference. */
int bc_attention_partial(const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                         const void* v_res, int batch, int n_heads, int n_kv_heads, int seq_len,
                         int kv_stride, int head_dim, void* workspace, size_t workspace_bytes,
                         void* stream);
int bc_attention_combine(const void* workspace, void* out, int batch, int n_heads, int n_kv_heads,
                         int seq_len, int head_dim, void* stream);

/* Per-head binary / compensated dispatch in one launch over a compensated cache:
 * head (b, h) is attended like bc_attention_gqa with k_res/v_res NULL where
 * modes[b*n_heads + h] == 0 and with them otherwise (modes as written by
 * bc_adaptive_select from bc_compute_head_entropy).  The reference's intent
 * for adaptive precision (src/adaptive_precision.cuh:6-49), which its demo
 * dispatches per layer in Python (examples/generation_demo.py:129-141).
 * head_dim a multiple of 32 up to 256 (the matrix-core kernel at 64, 128 and
 * 256, the VALU kernel otherwise); workspace as bc_attention_workspace_size. */
int bc_head_mode_attention(const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                           const void* v_res, const uint8_t* modes, void* out, int batch,
                           int n_heads, int n_kv_heads, int seq_len, int kv_stride, int head_dim,
                           void* workspace, size_t workspace_bytes, void* stream);

/* One decode step on ring caches of capacity batch*n_kv_heads*max_seq: the new
 * token k_new / v_new ([batch*n_kv_heads, head_dim] fp16) is encoded into
 * position current_len % max_seq of every (b, kv head) row with the
 * online-encode math, then q attends over the min(current_len + 1, max_seq)
 * filled positions.  Same cache bytes and output as bc_online_encode_kv
 * followed by bc_attention_gqa (seq_len = min(current_len + 1, max_seq),
 * kv_stride = max_seq), and the same workspace; one launch fewer when the
 * matrix-core kernel runs with one query-head group per kv head.  Replaces
 * the pair online_encode_token (src/online_encode.cu:122-149) +
 * compensated_attention (src/compensated_attention.cu:111-134) that
 * BitCache.append / attend issue (bitcache/__init__.py:95-148).  k_res/v_res
 * NULL: binary caches and binary attention. */
int bc_append_attention(const void* q, const void* k_new, const void* v_new, void* k_bin,
                        void* k_res, void* v_bin, void* v_res, void* out, int batch, int n_heads,
                        int n_kv_heads, int head_dim, int64_t current_len, int max_seq,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Per-key binary scores xnor_dot * 1/sqrt(d) (float32 [batch, n_heads, seq_len])
 * and/or the XNOR popcounts (int32, same shape); either output may be NULL.
 * Bit-exact.  Exposes the score of src/xnor_dot.cuh:14-31 /
 * src/binary_attention.cu:56, :63 (computed there but never returned). */
int bc_binary_scores(const void* q, const void* k_bin, float* scores, int32_t* popcounts,
                     int batch, int n_heads, int n_kv_heads, int seq_len, int kv_stride,
                     int head_dim, void* stream);

/* Per-(b,h) Shannon entropy of the softmax over binary scores (no 1/sqrt(d)).
 * Replaces launch_compute_head_entropy (src/adaptive_precision.cu:146-169). */
int bc_compute_head_entropy(const void* q, const void* k_bin, float* entropy, int batch,
                            int n_heads, int seq_len, int head_dim, void* stream);

/* General form of bc_compute_head_entropy: GQA (query head h reads kv head
 * h / (n_heads / n_kv_heads)) and a ring-buffer stride (blob capacity
 * batch*n_kv_heads*kv_stride, keys [0, seq_len) valid), so that the entropy of
 * a partly filled ring cache can be taken.  No counterpart in the reference
 * (which assumes n_kv_heads == n_heads and kv_stride == seq_len). */
int bc_compute_head_entropy_gqa(const void* q, const void* k_bin, float* entropy, int batch,
                                int n_heads, int n_kv_heads, int seq_len, int kv_stride,
                                int head_dim, void* stream);

/* bc_compute_head_entropy_gqa over several blocks per head: each block takes a
 * key chunk and leaves its (max, sum e, sum e*s) in the workspace, and a second
 * launch merges them (the single-block entry points keep one block per head,
 * which cannot draw a CU's share of HBM bandwidth).  Workspace bytes from
 * bc_entropy_workspace_size (0: the shape runs one block per head; a NULL
 * workspace selects the single-block kernel).  Same entropies to fp32
 * rounding.  No counterpart in the reference. */
int bc_entropy_workspace_size(int batch, int n_heads, int seq_len, size_t* bytes);
int bc_compute_head_entropy_ws(const void* q, const void* k_bin, float* entropy, int batch,
                               int n_heads, int n_kv_heads, int seq_len, int kv_stride,
                               int head_dim, void* workspace, size_t workspace_bytes, void* stream);

/* mode[i] = entropy[i] >= threshold ? 0 (binary) : 1 (compensated).
 * Replaces launch_adaptive_select (src/adaptive_precision.cu:171-186). */
int bc_adaptive_select(const float* entropy, uint8_t* modes, int batch, int n_heads,
                       float threshold, void* stream);

/* Adaptive precision: per (b, query head) the top_k keys by the exact binary
 * key scale_k*(2*popcount-d) (ties: lowest index) use the compensated score
 * and V; the others use binary score and V; one softmax over all keys.
 * selected (optional, uint8 [batch, n_heads, seq_len]) receives the 0/1 set.
 * seq_len up to 2^26 (BC_ERR_UNSUPPORTED above).  The workspace holds about
 * 5 bytes per query head and key (selection lists and popcounts) plus the
 * attention partials.
 * No counterpart in the reference (its intent: src/adaptive_precision.cuh:6-12). */
int bc_adaptive_attention_workspace_size(int batch, int n_heads, int n_kv_heads, int seq_len,
                                         int head_dim, size_t* bytes);
int bc_adaptive_attention(const void* q, const void* k_bin, const void* k_res, const void* v_bin,
                          const void* v_res, void* out, uint8_t* selected, int batch,
                          int n_heads, int n_kv_heads, int seq_len, int kv_stride, int head_dim,
                          int top_k, void* workspace, size_t workspace_bytes, void* stream);

/* Exact fp16 attention with fp32 accumulation over dense K/V
 * [batch, n_kv_heads, seq_len, head_dim] (the speed baseline and GPU oracle).
 * Workspace from bc_attention_workspace_size().
 * Replaces launch_reference_attention (src/reference_attention.cu:71-91). */
int bc_reference_attention(const void* q, const void* k, const void* v, void* out, int batch,
                           int n_heads, int n_kv_heads, int seq_len, int head_dim,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ---- format conversion -------------------------------------------------------- */
/* Dense planar blob (capacity n) <-> reference array-of-structs bytes
 * (BinaryVec: u32 words[8] + fp16 scale + pad = 36 B; ResidualVec: u8[128] + fp16 = 130 B;
 * src/binary_encode.cuh:13-18, src/residual.cuh:11-16).  Unused tail bytes of
 * each reference struct are written as zero. */
int bc_binary_to_reference(const void* blob, void* ref_aos, int64_t n, int head_dim, void* stream);
int bc_binary_from_reference(const void* ref_aos, void* blob, int64_t n, int head_dim,
                             void* stream);
int bc_residual_to_reference(const void* blob, void* ref_aos, int64_t n, int head_dim,
                             void* stream);
int bc_residual_from_reference(const void* ref_aos, void* blob, int64_t n, int head_dim,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BITCACHE_H_ */

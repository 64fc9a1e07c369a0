// bitcache_amd._C: thin PyTorch-ROCm extension over the C ABI (include/bitcache.h).
//
// Keeps the operator names and argument orders of the reference module
// bitcache._C (src/torch_binding.cpp:168-177) and adds the GQA / ring-stride /
// adaptive / fused-encode operators.  Each op validates its tensors, allocates
// outputs (and split-KV workspaces) through PyTorch's caching allocator and
// calls the C ABI on the current HIP stream; a non-zero status becomes a
// RuntimeError carrying bc_last_error().
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <optional>
#include <tuple>

#include "bitcache.h"

namespace {

#define BC_CHECK_DEV(x) TORCH_CHECK((x).device().is_cuda(), #x " must be a ROCm (cuda) tensor")
#define BC_CHECK_CONTIG(x) TORCH_CHECK((x).is_contiguous(), #x " must be contiguous")
#define BC_CHECK_HALF(x) TORCH_CHECK((x).scalar_type() == torch::kFloat16, #x " must be float16")
#define BC_CHECK_U8(x) TORCH_CHECK((x).scalar_type() == torch::kUInt8, #x " must be uint8")
#define BC_CHECK_INPUT(x) \
    BC_CHECK_DEV(x);      \
    BC_CHECK_CONTIG(x);   \
    BC_CHECK_HALF(x)
#define BC_CHECK_BLOB(x) \
    BC_CHECK_DEV(x);     \
    BC_CHECK_CONTIG(x);  \
    BC_CHECK_U8(x)

void check_status(int st, const char* op) {
    TORCH_CHECK(st == BC_OK, "bitcache ", op, " failed (", bc_status_string(st), "): ", bc_last_error());
}

void* stream_of(const torch::Tensor& t) {
    return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_same_device(const torch::Tensor& a, const torch::Tensor& b, const char* name) {
    TORCH_CHECK(a.device() == b.device(), name, " must be on the same device as the query/input");
}

// ------------------------------------------------------------------ blob capacity
// The planar layout puts a blob's scale plane at capacity * d/8 (binary) or
// capacity * d/2 (residual) bytes, so every op must know the capacity a blob
// was written with: the size of the allocation it lives in.
//  - A tensor that starts at its storage's first byte but covers less of it is
//    a prefix view of a whole blob, as the reference's BitCache.attend slices
//    its ring buffers (bitcache/__init__.py:134-139): capacity = storage bytes.
//  - Any other tensor (a whole allocation, or a view at an offset into a
//    caller's pool) is a blob of its own: capacity = numel / bytes per vector.
struct Blob {
    void* base;
    int64_t cap;
};

Blob resolve_blob(const torch::Tensor& t, int64_t per, const char* name) {
    TORCH_CHECK(t.device().is_cuda(), name, " must be a ROCm (cuda) tensor");
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
    TORCH_CHECK(t.scalar_type() == torch::kUInt8, name, " must be uint8");
    const int64_t stor = (int64_t)t.storage().nbytes();
    const bool prefix = t.storage_offset() == 0 && t.numel() < stor;
    const int64_t bytes = prefix ? stor : t.numel();
    TORCH_CHECK(bytes % per == 0, name, ": ", bytes, prefix ? " bytes of storage" : " bytes",
                " is not a whole number of ", per, "-byte vectors");
    return Blob{t.data_ptr(), bytes / per};
}

// A blob whose capacity must be exactly `vecs` vectors (the layout the op reads or writes).
void* blob_exact(const torch::Tensor& t, int64_t vecs, int64_t per, const char* name) {
    const Blob b = resolve_blob(t, per, name);
    TORCH_CHECK(b.cap == vecs, name, " holds ", b.cap, " vectors of ", per, " bytes but this shape"
                " needs a blob of exactly ", vecs, " (its planes are laid out for its capacity)");
    return b.base;
}

// Reference-signature attention ops (src/torch_binding.cpp:68-117, :141-162)
// take no stride: keys of row r = b*n_heads + h are read at r*kv_stride + s
// with kv_stride = capacity / (batch*n_heads).  A blob of exactly
// batch*n_heads*seq_len vectors gives kv_stride = seq_len (the reference's
// reading); a prefix view of a ring of max_seq slots per row gives
// kv_stride = max_seq, the stride the ring was written with
// (src/online_encode.cu:139), so a partly filled ring reads its own slots.
int64_t ref_kv_stride(const Blob& b, int64_t batch, int64_t n_heads, int64_t seq_len,
                      const char* name) {
    const int64_t rows = batch * n_heads;
    if (rows == 0) return seq_len;
    TORCH_CHECK(b.cap % rows == 0 && b.cap / rows >= seq_len && b.cap / rows <= INT32_MAX, name,
                " holds ", b.cap, " vectors: not batch*n_heads*kv_stride (batch*n_heads = ", rows,
                ") with kv_stride >= seq_len = ", seq_len);
    return b.cap / rows;
}

// ------------------------------------------------------------------ encode
torch::Tensor binary_encode(torch::Tensor src) {
    BC_CHECK_INPUT(src);
    TORCH_CHECK(src.dim() == 2, "src must be 2D [n_vecs, head_dim]");
    const int64_t n = src.size(0);
    const int64_t d = src.size(1);
    TORCH_CHECK(d % 32 == 0, "head_dim must be a multiple of 32");
    TORCH_CHECK(d <= 256, "head_dim exceeds MAX_HEAD_DIM=256");
    c10::DeviceGuard guard(src.device());
    auto out = torch::empty({n * bc_sizeof_binary_vec()},
                            torch::TensorOptions().dtype(torch::kUInt8).device(src.device()));
    check_status(bc_binary_encode(src.data_ptr(), out.data_ptr(), n, (int)d, stream_of(src)),
                 "binary_encode");
    return out;
}

torch::Tensor residual_encode(torch::Tensor src, torch::Tensor binary_blob) {
    BC_CHECK_INPUT(src);
    BC_CHECK_BLOB(binary_blob);
    check_same_device(src, binary_blob, "binary_blob");
    TORCH_CHECK(src.dim() == 2, "src must be 2D [n_vecs, head_dim]");
    const int64_t n = src.size(0);
    const int64_t d = src.size(1);
    TORCH_CHECK(d % 32 == 0, "head_dim must be a multiple of 32");
    TORCH_CHECK(d <= 256, "head_dim exceeds MAX_HEAD_DIM=256");
    void* bin = blob_exact(binary_blob, n, bc_sizeof_binary_vec(), "binary_blob");
    c10::DeviceGuard guard(src.device());
    auto out = torch::empty({n * bc_sizeof_residual_vec()},
                            torch::TensorOptions().dtype(torch::kUInt8).device(src.device()));
    check_status(bc_residual_encode(src.data_ptr(), bin, out.data_ptr(), n,
                                    (int)d, stream_of(src)),
                 "residual_encode");
    return out;
}

std::tuple<torch::Tensor, torch::Tensor> encode_fused(torch::Tensor src, bool fp32_scale) {
    BC_CHECK_INPUT(src);
    TORCH_CHECK(src.dim() == 2, "src must be 2D [n_vecs, head_dim]");
    const int64_t n = src.size(0);
    const int64_t d = src.size(1);
    TORCH_CHECK(d % 32 == 0 && d <= 256, "head_dim must be a multiple of 32 and <= 256");
    c10::DeviceGuard guard(src.device());
    auto opts = torch::TensorOptions().dtype(torch::kUInt8).device(src.device());
    auto bin = torch::empty({n * bc_sizeof_binary_vec()}, opts);
    auto res = torch::empty({n * bc_sizeof_residual_vec()}, opts);
    check_status(bc_encode_fused(src.data_ptr(), bin.data_ptr(), res.data_ptr(), n, (int)d,
                                 fp32_scale ? 1 : 0, stream_of(src)),
                 "encode_fused");
    return {bin, res};
}

// The memory floor of encode_fused: same kernel, loads and stores, no
// arithmetic; bin / res are blobs of capacity n_vecs (their bytes become
// meaningless).
void encode_traffic_probe(torch::Tensor src, torch::Tensor bin, torch::Tensor res) {
    BC_CHECK_INPUT(src);
    TORCH_CHECK(src.dim() == 2, "src must be 2D [n_vecs, head_dim]");
    const int64_t n = src.size(0);
    const int64_t d = src.size(1);
    TORCH_CHECK(bin.is_cuda() && res.is_cuda() && bin.is_contiguous() && res.is_contiguous() &&
                    bin.dtype() == torch::kUInt8 && res.dtype() == torch::kUInt8,
                "bin / res must be contiguous uint8 device tensors");
    TORCH_CHECK(bin.numel() == n * bc_sizeof_binary_vec() && res.numel() == n * bc_sizeof_residual_vec(),
                "bin / res must be blobs of capacity n_vecs");
    c10::DeviceGuard guard(src.device());
    check_status(bc_encode_traffic_probe(src.data_ptr(), bin.data_ptr(), res.data_ptr(), n, (int)d,
                                         stream_of(src)),
                 "encode_traffic_probe");
}

// The device's streaming-read ceiling: reads src's bytes once (measurement
// aid); returns the output words, of which the first 4 per workgroup (four
// workgroups per CU, at most one per 16 bytes) hold the per-wave XORs
torch::Tensor read_probe(torch::Tensor src) {
    TORCH_CHECK(src.is_cuda() && src.is_contiguous(), "src must be a contiguous device tensor");
    const int64_t n = src.numel() * src.element_size();
    TORCH_CHECK(n % 16 == 0, "src must hold a multiple of 16 bytes");
    c10::DeviceGuard guard(src.device());
    auto out = torch::empty({BC_READ_PROBE_OUT_WORDS}, src.options().dtype(torch::kInt32));
    check_status(bc_read_probe(src.data_ptr(), n, out.data_ptr(), stream_of(src)), "read_probe");
    return out;
}

// One mixed stream: reads 3 * dst's bytes of src, writes dst (bc_mix_probe).
void mix_probe(torch::Tensor src, torch::Tensor dst, bool nt_store) {
    TORCH_CHECK(src.is_cuda() && src.is_contiguous() && dst.is_cuda() && dst.is_contiguous(),
                "src and dst must be contiguous device tensors");
    check_same_device(src, dst, "dst");
    const int64_t nw = dst.numel() * dst.element_size();
    TORCH_CHECK(src.numel() * src.element_size() >= 3 * nw, "src must hold 3x dst's bytes");
    c10::DeviceGuard guard(src.device());
    check_status(bc_mix_probe(src.data_ptr(), dst.data_ptr(), nw, nt_store ? 1 : 0, stream_of(src)),
                 "mix_probe");
}

void check_kv_token(const torch::Tensor& kv, int64_t batch, int64_t n_heads, int64_t d) {
    BC_CHECK_INPUT(kv);
    TORCH_CHECK(kv.numel() == batch * n_heads * d, "kv must hold batch*n_heads*head_dim values");
}

// A residual cache that is the binary cache itself (the reference's binary-mode
// BitCache passes _k_bin twice, bitcache/__init__.py:104-111) means a binary-only
// cache: nothing is written as residual (the reference's kernel wrote 130-byte
// residual records into the 36-byte-per-slot buffer).
void online_encode_token(torch::Tensor kv, torch::Tensor binary_cache,
                         std::optional<torch::Tensor> residual_cache, int64_t batch,
                         int64_t n_heads, int64_t head_dim, int64_t current_len, int64_t max_seq) {
    check_kv_token(kv, batch, n_heads, head_dim);
    check_same_device(kv, binary_cache, "binary_cache");
    TORCH_CHECK(max_seq > 0, "max_seq must be > 0");
    const int64_t cap = batch * n_heads * max_seq;
    void* bin = blob_exact(binary_cache, cap, bc_sizeof_binary_vec(), "binary_cache");
    void* res = nullptr;
    if (residual_cache.has_value() && !residual_cache->is_alias_of(binary_cache)) {
        check_same_device(kv, *residual_cache, "residual_cache");
        res = blob_exact(*residual_cache, cap, bc_sizeof_residual_vec(), "residual_cache");
    }
    c10::DeviceGuard guard(kv.device());
    check_status(bc_online_encode_token(kv.data_ptr(), bin, res, (int)batch,
                                        (int)n_heads, (int)head_dim, current_len, (int)max_seq,
                                        stream_of(kv)),
                 "online_encode_token");
}

void online_encode_kv(torch::Tensor k, torch::Tensor v, torch::Tensor k_bin,
                      std::optional<torch::Tensor> k_res, torch::Tensor v_bin,
                      std::optional<torch::Tensor> v_res, int64_t batch, int64_t n_heads,
                      int64_t head_dim, int64_t current_len, int64_t max_seq) {
    check_kv_token(k, batch, n_heads, head_dim);
    check_kv_token(v, batch, n_heads, head_dim);
    TORCH_CHECK(max_seq > 0, "max_seq must be > 0");
    const int64_t cap = batch * n_heads * max_seq;
    void* kb = blob_exact(k_bin, cap, bc_sizeof_binary_vec(), "k_bin");
    void* vb = blob_exact(v_bin, cap, bc_sizeof_binary_vec(), "v_bin");
    TORCH_CHECK(k_res.has_value() == v_res.has_value(), "k_res and v_res: both or neither");
    void *kr = nullptr, *vr = nullptr;
    if (k_res.has_value()) {
        kr = blob_exact(*k_res, cap, bc_sizeof_residual_vec(), "k_res");
        vr = blob_exact(*v_res, cap, bc_sizeof_residual_vec(), "v_res");
    }
    c10::DeviceGuard guard(k.device());
    check_status(bc_online_encode_kv(k.data_ptr(), v.data_ptr(), kb, kr, vb, vr, (int)batch,
                                     (int)n_heads, (int)head_dim,
                                     current_len, (int)max_seq, stream_of(k)),
                 "online_encode_kv");
}

void encode_into_cache(torch::Tensor src, torch::Tensor binary_cache,
                       std::optional<torch::Tensor> residual_cache, int64_t rows, int64_t seq,
                       int64_t head_dim, int64_t start_pos, int64_t max_seq, bool fp32_scale) {
    BC_CHECK_INPUT(src);
    check_same_device(src, binary_cache, "binary_cache");
    TORCH_CHECK(src.numel() == rows * seq * head_dim, "src must be [rows, seq, head_dim]");
    TORCH_CHECK(max_seq > 0 && start_pos >= 0 && start_pos + seq <= max_seq,
                "start_pos + seq must fit in max_seq");
    const int64_t cap = rows * max_seq;
    void* bin = blob_exact(binary_cache, cap, bc_sizeof_binary_vec(), "binary_cache");
    void* res = nullptr;
    if (residual_cache.has_value()) {
        check_same_device(src, *residual_cache, "residual_cache");
        res = blob_exact(*residual_cache, cap, bc_sizeof_residual_vec(), "residual_cache");
    }
    c10::DeviceGuard guard(src.device());
    check_status(bc_encode_into_cache(src.data_ptr(), bin, res, rows, (int)seq,
                                      (int)head_dim, (int)start_pos, (int)max_seq,
                                      fp32_scale ? 1 : 0, stream_of(src)),
                 "encode_into_cache");
}

// [batch, seq, n_heads, head_dim] source (bc_encode_into_cache_bshd)
void encode_into_cache_bshd(torch::Tensor src, torch::Tensor binary_cache,
                            std::optional<torch::Tensor> residual_cache, int64_t batch, int64_t seq,
                            int64_t n_heads, int64_t head_dim, int64_t start_pos, int64_t max_seq,
                            bool fp32_scale) {
    BC_CHECK_INPUT(src);
    check_same_device(src, binary_cache, "binary_cache");
    TORCH_CHECK(src.numel() == batch * seq * n_heads * head_dim,
                "src must be [batch, seq, n_heads, head_dim]");
    TORCH_CHECK(max_seq > 0 && start_pos >= 0 && start_pos + seq <= max_seq,
                "start_pos + seq must fit in max_seq");
    const int64_t cap = batch * n_heads * max_seq;
    void* bin = blob_exact(binary_cache, cap, bc_sizeof_binary_vec(), "binary_cache");
    void* res = nullptr;
    if (residual_cache.has_value()) {
        check_same_device(src, *residual_cache, "residual_cache");
        res = blob_exact(*residual_cache, cap, bc_sizeof_residual_vec(), "residual_cache");
    }
    c10::DeviceGuard guard(src.device());
    check_status(bc_encode_into_cache_bshd(src.data_ptr(), bin, res, (int)batch, (int)seq,
                                           (int)n_heads, (int)head_dim, (int)start_pos,
                                           (int)max_seq, fp32_scale ? 1 : 0, stream_of(src)),
                 "encode_into_cache_bshd");
}

// ------------------------------------------------------------------ attention
void check_q(const torch::Tensor& Q, int64_t batch, int64_t n_heads, int64_t d) {
    BC_CHECK_INPUT(Q);
    TORCH_CHECK(Q.numel() == batch * n_heads * d, "Q must hold batch*n_heads*head_dim values, got ",
                Q.numel());
}

torch::Tensor workspace_for(const torch::Tensor& Q, size_t bytes) {
    return torch::empty({(int64_t)(bytes > 0 ? bytes : 1)},
                        torch::TensorOptions().dtype(torch::kUInt8).device(Q.device()));
}

// The four cache blobs of an attention call, each of capacity exactly `cap`
// vectors; residual pointers are null when the residual blobs are absent.
struct CachePtrs {
    void *kb, *kr, *vb, *vr;
};

CachePtrs cache_blobs(const torch::Tensor& Q, const torch::Tensor& K_bin,
                      const std::optional<torch::Tensor>& K_res, const torch::Tensor& V_bin,
                      const std::optional<torch::Tensor>& V_res, int64_t cap) {
    check_same_device(Q, K_bin, "K_bin");
    check_same_device(Q, V_bin, "V_bin");
    CachePtrs c{};
    c.kb = blob_exact(K_bin, cap, bc_sizeof_binary_vec(), "K_bin");
    c.vb = blob_exact(V_bin, cap, bc_sizeof_binary_vec(), "V_bin");
    TORCH_CHECK(K_res.has_value() == V_res.has_value(), "K_res and V_res: both or neither");
    if (K_res.has_value()) {
        check_same_device(Q, *K_res, "K_res");
        check_same_device(Q, *V_res, "V_res");
        c.kr = blob_exact(*K_res, cap, bc_sizeof_residual_vec(), "K_res");
        c.vr = blob_exact(*V_res, cap, bc_sizeof_residual_vec(), "V_res");
    }
    return c;
}

void check_heads(int64_t n_heads, int64_t n_kv_heads, int64_t seq_len, int64_t kv_stride) {
    TORCH_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                "n_heads must be a multiple of n_kv_heads");
    TORCH_CHECK(kv_stride >= seq_len, "kv_stride must be >= seq_len");
}

torch::Tensor attention(torch::Tensor Q, torch::Tensor K_bin, std::optional<torch::Tensor> K_res,
                        torch::Tensor V_bin, std::optional<torch::Tensor> V_res, int64_t batch,
                        int64_t n_heads, int64_t n_kv_heads, int64_t seq_len, int64_t kv_stride,
                        int64_t head_dim) {
    check_q(Q, batch, n_heads, head_dim);
    check_heads(n_heads, n_kv_heads, seq_len, kv_stride);
    const CachePtrs c = cache_blobs(Q, K_bin, K_res, V_bin, V_res, batch * n_kv_heads * kv_stride);
    c10::DeviceGuard guard(Q.device());
    size_t ws_bytes = 0;
    check_status(bc_attention_workspace_size((int)batch, (int)n_heads, (int)n_kv_heads,
                                             (int)seq_len, (int)head_dim, &ws_bytes),
                 "attention_workspace_size");
    auto ws = workspace_for(Q, ws_bytes);
    auto out = torch::empty({batch, n_heads, head_dim}, Q.options());
    check_status(bc_attention_gqa(Q.data_ptr(), c.kb, c.kr, c.vb, c.vr, out.data_ptr(), (int)batch,
                                  (int)n_heads, (int)n_kv_heads, (int)seq_len, (int)kv_stride,
                                  (int)head_dim, ws.data_ptr(), ws_bytes, stream_of(Q)),
                 "attention");
    return out.view(Q.sizes());
}

// Per-head binary / compensated dispatch in one launch (bc_head_mode_attention):
// modes uint8 [batch, n_heads], 0 = binary for that head.
torch::Tensor head_mode_attention(torch::Tensor Q, torch::Tensor K_bin, torch::Tensor K_res,
                                  torch::Tensor V_bin, torch::Tensor V_res, torch::Tensor modes,
                                  int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                                  int64_t seq_len, int64_t kv_stride, int64_t head_dim) {
    check_q(Q, batch, n_heads, head_dim);
    BC_CHECK_DEV(modes);
    BC_CHECK_CONTIG(modes);
    BC_CHECK_U8(modes);
    check_same_device(Q, modes, "modes");
    TORCH_CHECK(modes.numel() == batch * n_heads, "modes must hold batch*n_heads values");
    check_heads(n_heads, n_kv_heads, seq_len, kv_stride);
    const CachePtrs c = cache_blobs(Q, K_bin, K_res, V_bin, V_res, batch * n_kv_heads * kv_stride);
    c10::DeviceGuard guard(Q.device());
    size_t ws_bytes = 0;
    check_status(bc_attention_workspace_size((int)batch, (int)n_heads, (int)n_kv_heads,
                                             (int)seq_len, (int)head_dim, &ws_bytes),
                 "attention_workspace_size");
    auto ws = workspace_for(Q, ws_bytes);
    auto out = torch::empty({batch, n_heads, head_dim}, Q.options());
    check_status(bc_head_mode_attention(Q.data_ptr(), c.kb, c.kr, c.vb, c.vr,
                                        modes.data_ptr<uint8_t>(), out.data_ptr(), (int)batch,
                                        (int)n_heads, (int)n_kv_heads, (int)seq_len, (int)kv_stride,
                                        (int)head_dim, ws.data_ptr(), ws_bytes, stream_of(Q)),
                 "head_mode_attention");
    return out.view(Q.sizes());
}

// One decode step: append the token (k, v: [batch*n_kv_heads*head_dim] fp16) at
// position current_len % max_seq of the ring caches, then attend over the
// filled positions (bc_append_attention).
torch::Tensor append_attention(torch::Tensor Q, torch::Tensor k, torch::Tensor v,
                               torch::Tensor K_bin, std::optional<torch::Tensor> K_res,
                               torch::Tensor V_bin, std::optional<torch::Tensor> V_res,
                               int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                               int64_t head_dim, int64_t current_len, int64_t max_seq) {
    check_q(Q, batch, n_heads, head_dim);
    TORCH_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                "n_heads must be a multiple of n_kv_heads");
    check_kv_token(k, batch, n_kv_heads, head_dim);
    check_kv_token(v, batch, n_kv_heads, head_dim);
    check_same_device(Q, k, "k");
    check_same_device(Q, v, "v");
    TORCH_CHECK(max_seq > 0 && current_len >= 0, "max_seq must be > 0 and current_len >= 0");
    const CachePtrs c = cache_blobs(Q, K_bin, K_res, V_bin, V_res, batch * n_kv_heads * max_seq);
    c10::DeviceGuard guard(Q.device());
    const int64_t seq_len = current_len + 1 < max_seq ? current_len + 1 : max_seq;
    size_t ws_bytes = 0;
    check_status(bc_attention_workspace_size((int)batch, (int)n_heads, (int)n_kv_heads,
                                             (int)seq_len, (int)head_dim, &ws_bytes),
                 "attention_workspace_size");
    auto ws = workspace_for(Q, ws_bytes);
    auto out = torch::empty({batch, n_heads, head_dim}, Q.options());
    check_status(bc_append_attention(Q.data_ptr(), k.data_ptr(), v.data_ptr(), c.kb, c.kr, c.vb,
                                     c.vr, out.data_ptr(), (int)batch, (int)n_heads,
                                     (int)n_kv_heads, (int)head_dim, current_len, (int)max_seq,
                                     ws.data_ptr(), ws_bytes, stream_of(Q)),
                 "append_attention");
    return out.view(Q.sizes());
}

// Phase 1 only: returns the workspace holding the split partials.
torch::Tensor attention_partial(torch::Tensor Q, torch::Tensor K_bin,
                                std::optional<torch::Tensor> K_res, torch::Tensor V_bin,
                                std::optional<torch::Tensor> V_res, int64_t batch, int64_t n_heads,
                                int64_t n_kv_heads, int64_t seq_len, int64_t kv_stride,
                                int64_t head_dim) {
    check_q(Q, batch, n_heads, head_dim);
    check_heads(n_heads, n_kv_heads, seq_len, kv_stride);
    const CachePtrs c = cache_blobs(Q, K_bin, K_res, V_bin, V_res, batch * n_kv_heads * kv_stride);
    c10::DeviceGuard guard(Q.device());
    size_t ws_bytes = 0;
    check_status(bc_attention_workspace_size((int)batch, (int)n_heads, (int)n_kv_heads,
                                             (int)seq_len, (int)head_dim, &ws_bytes),
                 "attention_workspace_size");
    auto ws = workspace_for(Q, ws_bytes);
    check_status(bc_attention_partial(Q.data_ptr(), c.kb, c.kr, c.vb, c.vr, (int)batch,
                                      (int)n_heads, (int)n_kv_heads, (int)seq_len, (int)kv_stride,
                                      (int)head_dim, ws.data_ptr(), ws_bytes, stream_of(Q)),
                 "attention_partial");
    return ws;
}

torch::Tensor attention_combine(torch::Tensor ws, int64_t batch, int64_t n_heads,
                                int64_t n_kv_heads, int64_t seq_len, int64_t head_dim) {
    BC_CHECK_DEV(ws);
    BC_CHECK_CONTIG(ws);
    size_t need = 0;
    check_status(bc_attention_workspace_size((int)batch, (int)n_heads, (int)n_kv_heads,
                                             (int)seq_len, (int)head_dim, &need),
                 "attention_workspace_size");
    TORCH_CHECK((size_t)ws.numel() * ws.element_size() >= need, "workspace too small");
    c10::DeviceGuard guard(ws.device());
    auto out = torch::empty({batch, n_heads, head_dim},
                            torch::TensorOptions().dtype(torch::kFloat16).device(ws.device()));
    check_status(bc_attention_combine(ws.data_ptr(), out.data_ptr(), (int)batch, (int)n_heads,
                                      (int)n_kv_heads, (int)seq_len, (int)head_dim, stream_of(ws)),
                 "attention_combine");
    return out;
}

// Reference signatures (src/torch_binding.cpp:68-117): MHA; the stride of the
// rows comes from the blob's capacity (ref_kv_stride), so the prefix views the
// reference's BitCache passes read the slots it wrote.
torch::Tensor binary_attention(torch::Tensor Q, torch::Tensor K_bin, torch::Tensor V_bin,
                               int64_t batch, int64_t n_heads, int64_t seq_len, int64_t head_dim) {
    const int64_t stride = ref_kv_stride(resolve_blob(K_bin, bc_sizeof_binary_vec(), "K_bin"),
                                         batch, n_heads, seq_len, "K_bin");
    return attention(Q, K_bin, std::nullopt, V_bin, std::nullopt, batch, n_heads, n_heads, seq_len,
                     stride, head_dim);
}

torch::Tensor compensated_attention(torch::Tensor Q, torch::Tensor K_bin, torch::Tensor K_res,
                                    torch::Tensor V_bin, torch::Tensor V_res, int64_t batch,
                                    int64_t n_heads, int64_t seq_len, int64_t head_dim) {
    const int64_t stride = ref_kv_stride(resolve_blob(K_bin, bc_sizeof_binary_vec(), "K_bin"),
                                         batch, n_heads, seq_len, "K_bin");
    return attention(Q, K_bin, K_res, V_bin, V_res, batch, n_heads, n_heads, seq_len, stride,
                     head_dim);
}

std::tuple<torch::Tensor, torch::Tensor> adaptive_attention(
    torch::Tensor Q, torch::Tensor K_bin, torch::Tensor K_res, torch::Tensor V_bin,
    torch::Tensor V_res, int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t seq_len,
    int64_t kv_stride, int64_t head_dim, int64_t top_k, bool return_selected) {
    check_q(Q, batch, n_heads, head_dim);
    check_heads(n_heads, n_kv_heads, seq_len, kv_stride);
    TORCH_CHECK(top_k >= 0, "top_k must be >= 0");
    const CachePtrs c = cache_blobs(Q, K_bin, K_res, V_bin, V_res, batch * n_kv_heads * kv_stride);
    c10::DeviceGuard guard(Q.device());
    size_t ws_bytes = 0;
    check_status(bc_adaptive_attention_workspace_size((int)batch, (int)n_heads, (int)n_kv_heads,
                                                      (int)seq_len, (int)head_dim, &ws_bytes),
                 "adaptive_attention_workspace_size");
    auto ws = workspace_for(Q, ws_bytes);
    auto out = torch::empty({batch, n_heads, head_dim}, Q.options());
    torch::Tensor sel;
    uint8_t* selp = nullptr;
    if (return_selected) {
        sel = torch::empty({batch, n_heads, seq_len},
                           torch::TensorOptions().dtype(torch::kUInt8).device(Q.device()));
        selp = sel.data_ptr<uint8_t>();
    }
    check_status(bc_adaptive_attention(Q.data_ptr(), c.kb, c.kr, c.vb, c.vr, out.data_ptr(), selp,
                                       (int)batch, (int)n_heads, (int)n_kv_heads, (int)seq_len,
                                       (int)kv_stride, (int)head_dim, (int)top_k, ws.data_ptr(),
                                       ws_bytes, stream_of(Q)),
                 "adaptive_attention");
    return {out.view(Q.sizes()), sel};
}

std::tuple<torch::Tensor, torch::Tensor> binary_scores(torch::Tensor Q, torch::Tensor K_bin,
                                                       int64_t batch, int64_t n_heads,
                                                       int64_t n_kv_heads, int64_t seq_len,
                                                       int64_t kv_stride, int64_t head_dim) {
    check_q(Q, batch, n_heads, head_dim);
    check_same_device(Q, K_bin, "K_bin");
    check_heads(n_heads, n_kv_heads, seq_len, kv_stride);
    void* kb = blob_exact(K_bin, batch * n_kv_heads * kv_stride, bc_sizeof_binary_vec(), "K_bin");
    c10::DeviceGuard guard(Q.device());
    auto scores = torch::empty({batch, n_heads, seq_len}, Q.options().dtype(torch::kFloat32));
    auto pcs = torch::empty({batch, n_heads, seq_len}, Q.options().dtype(torch::kInt32));
    check_status(bc_binary_scores(Q.data_ptr(), kb, scores.data_ptr<float>(),
                                  pcs.data_ptr<int32_t>(), (int)batch, (int)n_heads,
                                  (int)n_kv_heads, (int)seq_len, (int)kv_stride, (int)head_dim,
                                  stream_of(Q)),
                 "binary_scores");
    return {scores, pcs};
}

// GQA / ring-stride form (bc_compute_head_entropy_ws).
torch::Tensor head_entropy(torch::Tensor Q, torch::Tensor K_bin, int64_t batch, int64_t n_heads,
                           int64_t n_kv_heads, int64_t seq_len, int64_t kv_stride,
                           int64_t head_dim) {
    check_q(Q, batch, n_heads, head_dim);
    check_same_device(Q, K_bin, "K_bin");
    check_heads(n_heads, n_kv_heads, seq_len, kv_stride);
    void* kb = blob_exact(K_bin, batch * n_kv_heads * kv_stride, bc_sizeof_binary_vec(), "K_bin");
    c10::DeviceGuard guard(Q.device());
    auto ent = torch::empty({batch, n_heads}, Q.options().dtype(torch::kFloat32));
    // the key-split pass (several blocks per head) with a workspace from the
    // caching allocator; the same result as the single-block entry points
    size_t ws_bytes = 0;
    check_status(bc_entropy_workspace_size((int)batch, (int)n_heads, (int)seq_len, &ws_bytes),
                 "entropy_workspace_size");
    auto ws = workspace_for(Q, ws_bytes);
    check_status(bc_compute_head_entropy_ws(Q.data_ptr(), kb, ent.data_ptr<float>(), (int)batch,
                                            (int)n_heads, (int)n_kv_heads, (int)seq_len,
                                            (int)kv_stride, (int)head_dim,
                                            ws_bytes ? ws.data_ptr() : nullptr, ws_bytes,
                                            stream_of(Q)),
                 "compute_head_entropy");
    return ent;
}

// Reference signature (src/torch_binding.cpp:141-162); stride as binary_attention.
torch::Tensor compute_head_entropy(torch::Tensor Q, torch::Tensor K_bin, int64_t batch,
                                   int64_t n_heads, int64_t seq_len, int64_t head_dim) {
    const int64_t stride = ref_kv_stride(resolve_blob(K_bin, bc_sizeof_binary_vec(), "K_bin"),
                                         batch, n_heads, seq_len, "K_bin");
    return head_entropy(Q, K_bin, batch, n_heads, n_heads, seq_len, stride, head_dim);
}

torch::Tensor adaptive_select(torch::Tensor entropy, double threshold) {
    BC_CHECK_DEV(entropy);
    BC_CHECK_CONTIG(entropy);
    TORCH_CHECK(entropy.scalar_type() == torch::kFloat32, "entropy must be float32");
    c10::DeviceGuard guard(entropy.device());
    auto modes = torch::empty(entropy.sizes(), entropy.options().dtype(torch::kUInt8));
    check_status(bc_adaptive_select(entropy.data_ptr<float>(), modes.data_ptr<uint8_t>(), 1,
                                    (int)entropy.numel(), (float)threshold, stream_of(entropy)),
                 "adaptive_select");
    return modes;
}

torch::Tensor reference_attention(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                  int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                                  int64_t seq_len, int64_t head_dim) {
    check_q(Q, batch, n_heads, head_dim);
    BC_CHECK_INPUT(K);
    BC_CHECK_INPUT(V);
    check_same_device(Q, K, "K");
    check_same_device(Q, V, "V");
    TORCH_CHECK(K.numel() == batch * n_kv_heads * seq_len * head_dim &&
                    V.numel() == K.numel(),
                "K/V must be [batch, n_kv_heads, seq_len, head_dim]");
    c10::DeviceGuard guard(Q.device());
    size_t ws_bytes = 0;
    check_status(bc_attention_workspace_size((int)batch, (int)n_heads, (int)n_kv_heads,
                                             (int)seq_len, (int)head_dim, &ws_bytes),
                 "attention_workspace_size");
    auto ws = workspace_for(Q, ws_bytes);
    auto out = torch::empty({batch, n_heads, head_dim}, Q.options());
    check_status(bc_reference_attention(Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(),
                                        (int)batch, (int)n_heads, (int)n_kv_heads, (int)seq_len,
                                        (int)head_dim, ws.data_ptr(), ws_bytes, stream_of(Q)),
                 "reference_attention");
    return out.view(Q.sizes());
}

// ------------------------------------------------------------------ format conversion
torch::Tensor convert(torch::Tensor blob, int64_t n, int64_t head_dim, bool residual, bool to_ref) {
    const int64_t per = residual ? bc_sizeof_residual_vec() : bc_sizeof_binary_vec();
    BC_CHECK_BLOB(blob);
    TORCH_CHECK(blob.numel() == n * per, "blob must hold n * ", per, " bytes");
    // a planar input is read at its capacity's plane offsets
    if (to_ref) blob_exact(blob, n, per, "blob");
    c10::DeviceGuard guard(blob.device());
    auto out = to_ref ? torch::empty({n * per}, blob.options()) : torch::zeros({n * per}, blob.options());
    int st;
    if (residual)
        st = to_ref ? bc_residual_to_reference(blob.data_ptr(), out.data_ptr(), n, (int)head_dim, stream_of(blob))
                    : bc_residual_from_reference(blob.data_ptr(), out.data_ptr(), n, (int)head_dim, stream_of(blob));
    else
        st = to_ref ? bc_binary_to_reference(blob.data_ptr(), out.data_ptr(), n, (int)head_dim, stream_of(blob))
                    : bc_binary_from_reference(blob.data_ptr(), out.data_ptr(), n, (int)head_dim, stream_of(blob));
    check_status(st, "convert");
    return out;
}

int64_t sizeof_binary_vec() { return bc_sizeof_binary_vec(); }
int64_t sizeof_residual_vec() { return bc_sizeof_residual_vec(); }

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    // reference operators (src/torch_binding.cpp:168-177)
    m.def("binary_encode", &binary_encode, "Encode fp16 vectors to binary (sign bits + scale)");
    m.def("residual_encode", &residual_encode, "INT4 residuals from fp16 and a binary encoding");
    m.def("binary_attention", &binary_attention, "Binary-only approximate attention");
    m.def("compensated_attention", &compensated_attention, "Residual-compensated binary attention");
    m.def("online_encode_token", &online_encode_token, "Fused single-token encode and cache append",
          py::arg("kv"), py::arg("binary_cache"), py::arg("residual_cache"), py::arg("batch"),
          py::arg("n_heads"), py::arg("head_dim"), py::arg("current_len"), py::arg("max_seq"));
    m.def("compute_head_entropy", &compute_head_entropy, "Per-head entropy of binary attention");
    m.def("head_entropy", &head_entropy, "Per-head entropy, GQA / ring-stride form");
    m.def("sizeof_binary_vec", &sizeof_binary_vec, "Bytes per vector of a binary blob (36)");
    m.def("sizeof_residual_vec", &sizeof_residual_vec, "Bytes per vector of a residual blob (130)");
    // extensions
    m.def("encode_fused", &encode_fused, "Binary + residual encode in one pass", py::arg("src"),
          py::arg("fp32_scale") = false);
    m.def("encode_traffic_probe", &encode_traffic_probe,
          "encode_fused's loads and stores without its arithmetic (memory floor)");
    m.def("read_probe", &read_probe, "One streaming read of a tensor's bytes (the read ceiling)");
    m.def("mix_probe", &mix_probe, "A 3:1 read/write stream (the encoders' mixed-traffic ceiling)",
          py::arg("src"), py::arg("dst"), py::arg("nt_store") = false);
    m.def("online_encode_kv", &online_encode_kv, "K and V token encode in one launch");
    m.def("encode_into_cache", &encode_into_cache, "Bulk prefill into ring caches");
    m.def("encode_into_cache_bshd", &encode_into_cache_bshd,
          "Bulk prefill into ring caches from a [batch, seq, heads, d] source");
    m.def("attention", &attention, "GQA / ring-stride binary or compensated attention");
    m.def("append_attention", &append_attention, "One decode step: ring-cache append + attention");
    m.def("head_mode_attention", &head_mode_attention, "Per-head binary / compensated attention");
    m.def("attention_partial", &attention_partial, "Split-KV partials (phase 1 of attention)");
    m.def("attention_combine", &attention_combine, "Merge split-KV partials (phase 2)");
    m.def("adaptive_attention", &adaptive_attention, "Top-k residual selection attention");
    m.def("binary_scores", &binary_scores, "Exact per-key binary scores and popcounts");
    m.def("adaptive_select", &adaptive_select, "entropy >= threshold ? 0 (binary) : 1");
    m.def("reference_attention", &reference_attention, "Exact fp16 attention (fp32 accumulation)");
    m.def("convert", &convert, "Dense planar blob <-> reference array-of-structs bytes");
}

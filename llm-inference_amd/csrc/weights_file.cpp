// weights.bin parsing and tensor layout (host code only).
//
// The file is what python/export_weights.py:51-134 of MarcVivas/llm-inference
// writes and what include/model.hpp:18-93 + device_weights.hpp:57-110 read: a
// 44-byte header, a uint32 tokenizer-JSON length and the JSON, zero padding to
// a 64-byte offset, then fp16 tensors in layer order.  The engine copies the
// whole payload into one device allocation and hands out pointers into it;
// the attention path's consumer is the fused QKV weight (q_proj, k_proj and
// v_proj adjacent), which the projections read as one [q_dim + 2 kv_dim][hidden]
// matrix (model_inference.hpp:268, :354).
//
// Everything here is 64-bit integer arithmetic with overflow checks; nothing
// touches the GPU, so the parse can run (and be tested) on a host without one.
#include <cstdint>
#include <cstring>

#include "../../include/attn_mi355x.h"

static_assert(sizeof(attn_model_config) == 44, "weights.bin header is 44 bytes");

namespace {

constexpr uint64_t kHeaderBytes = sizeof(attn_model_config);
constexpr uint64_t kTokLenBytes = sizeof(uint32_t);
constexpr uint64_t kAbsent = UINT64_MAX;

// Running element cursor over the payload; any overflow poisons it.
struct Cursor {
    uint64_t at = 0;
    bool overflow = false;

    uint64_t claim(uint64_t a, uint64_t b = 1) {
        uint64_t n = 0;
        if (__builtin_mul_overflow(a, b, &n)) overflow = true;
        const uint64_t start = at;
        if (__builtin_add_overflow(at, n, &at)) overflow = true;
        return start;
    }
};

// Per-layer offsets (relative to the layer's first element) and the layer size,
// in the exporter's order (export_weights.py:100-122).
bool layer_offsets(const attn_model_config& c, bool qk_norm, attn_weights_layout& o) {
    const uint64_t H = c.hidden_size, D = c.head_dim, I = c.intermediate_size;
    const uint64_t q_dim = uint64_t(c.num_heads) * D, kv_dim = uint64_t(c.num_kv_heads) * D;
    Cursor cur;
    o.input_norm = cur.claim(H);
    o.q_proj = cur.claim(q_dim, H);
    o.k_proj = cur.claim(kv_dim, H);
    o.v_proj = cur.claim(kv_dim, H);
    o.q_norm = qk_norm ? cur.claim(D) : kAbsent;
    o.k_norm = qk_norm ? cur.claim(D) : kAbsent;
    o.o_proj = cur.claim(H, q_dim);
    o.post_attn_norm = cur.claim(H);
    o.gate_proj = cur.claim(I, H);
    o.up_proj = cur.claim(I, H);
    o.down_proj = cur.claim(H, I);
    o.layer_elems = cur.at;
    return !cur.overflow;
}

// Whole-payload offsets; returns the element count or kAbsent on overflow.
uint64_t payload_offsets(const attn_model_config& c, bool qk_norm, attn_weights_layout& o) {
    if (!layer_offsets(c, qk_norm, o)) return kAbsent;
    const uint64_t V = c.vocab_size, H = c.hidden_size;
    Cursor cur;
    o.embedding = cur.claim(V, H);
    o.layer_base = cur.claim(o.layer_elems, c.num_layers);
    o.final_norm = cur.claim(H);
    o.lm_head = cur.claim(V, H);
    return cur.overflow ? kAbsent : cur.at;
}

}  // namespace

extern "C" {

int attn_weights_layout_for(const attn_model_config* config, uint64_t payload_bytes,
                            attn_weights_layout* out) {
    if (!config || !out) return (int)hipErrorInvalidValue;
    attn_weights_layout plain{}, normed{};
    const uint64_t n_plain = payload_offsets(*config, false, plain);
    const uint64_t n_normed = payload_offsets(*config, true, normed);
    if (n_plain == kAbsent || n_plain > UINT64_MAX / 2) return ATTN_WEIGHTS_SIZE_OVERFLOW;
    // a QK-norm checkpoint is recognised by its exact size; everything else is
    // read as the reference's DeviceWeights reads it
    const bool qk = n_normed != kAbsent && n_normed != n_plain && n_normed <= UINT64_MAX / 2 &&
                    payload_bytes == 2 * n_normed;
    attn_weights_layout& lay = qk ? normed : plain;
    lay.config = *config;
    lay.has_qk_norm = qk ? 1u : 0u;
    lay.weights_bytes = payload_bytes;
    lay.layout_bytes = 2 * (qk ? n_normed : n_plain);
    if (payload_bytes < lay.layout_bytes) return ATTN_WEIGHTS_PAYLOAD_SHORT;
    *out = lay;
    return 0;
}

int attn_weights_parse(const void* head, size_t head_bytes, uint64_t file_bytes,
                       attn_weights_layout* out) {
    if (!head || !out) return (int)hipErrorInvalidValue;
    const uint64_t need = file_bytes < kHeaderBytes + kTokLenBytes ? file_bytes
                                                                   : kHeaderBytes + kTokLenBytes;
    if (head_bytes < need) return (int)hipErrorInvalidValue;
    const auto* b = static_cast<const unsigned char*>(head);

    // model_config.hpp:33-43: size, then magic
    if (file_bytes < kHeaderBytes) return ATTN_WEIGHTS_SHORT_HEADER;
    attn_model_config cfg;
    std::memcpy(&cfg, b, sizeof cfg);
    if (std::memcmp(cfg.magic, "QWEN", 4) != 0) return ATTN_WEIGHTS_BAD_MAGIC;

    // model.hpp:45-70: tokenizer length and payload, then the 64-byte boundary
    if (file_bytes - kHeaderBytes < kTokLenBytes) return ATTN_WEIGHTS_NO_TOKENIZER_LENGTH;
    uint32_t tok_len;
    std::memcpy(&tok_len, b + kHeaderBytes, sizeof tok_len);
    const uint64_t tok_at = kHeaderBytes + kTokLenBytes;
    if (file_bytes - tok_at < tok_len) return ATTN_WEIGHTS_TOKENIZER_TRUNCATED;
    const uint64_t weights_offset = (tok_at + tok_len + 63) & ~uint64_t(63);

    // model.hpp:84-86
    if (file_bytes <= weights_offset) return ATTN_WEIGHTS_NO_PAYLOAD;

    attn_weights_layout lay;
    const int rc = attn_weights_layout_for(&cfg, file_bytes - weights_offset, &lay);
    if (rc != 0) return rc;
    lay.tokenizer_offset = tok_at;
    lay.tokenizer_bytes = tok_len;
    lay.weights_offset = weights_offset;
    *out = lay;
    return 0;
}

const char* attn_weights_error_string(int code) {
    switch (code) {
        case ATTN_WEIGHTS_SHORT_HEADER:
            return "Buffer too small for ModelConfig header (expected 44 bytes)";
        case ATTN_WEIGHTS_BAD_MAGIC:
            return "Invalid binary file: Magic number is not 'QWEN'";
        case ATTN_WEIGHTS_NO_TOKENIZER_LENGTH:
            return "Corrupted model file: Missing tokenizer length field";
        case ATTN_WEIGHTS_TOKENIZER_TRUNCATED:
            return "Corrupted model file: Tokenizer payload truncated";
        case ATTN_WEIGHTS_NO_PAYLOAD:
            return "Corrupted model file: Missing weight payload";
        case ATTN_WEIGHTS_PAYLOAD_SHORT:
            return "Corrupted model file: Weight payload smaller than the tensors of its header";
        case ATTN_WEIGHTS_SIZE_OVERFLOW:
            return "Invalid model file: Tensor sizes overflow 64 bits";
        default:
            return nullptr;
    }
}

}  // extern "C"

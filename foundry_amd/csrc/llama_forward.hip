// fh_llama_forward: the decoder's layer loop, issued from native code.
//
// LlamaModel::forward (src/models/llama/model.rs:92-121) with the layer body
// of LlamaDecoderLayer::forward (:254-280), the attention of
// LlamaAttention::forward (src/models/llama/attention.rs:72-132) and the MLP
// of LlamaMlp::forward (src/models/llama/mlp.rs:49-58), then the greedy pick
// of Decoder::step (src/generate/mod.rs:192-204). Each step is one of the
// library's ops, called as a host would call it, so the results are those of
// the op-by-op sequence; what this saves is the host's per-op cost (argument
// marshalling in an interpreted caller), which bounds an eager prefill whose
// kernels take a few microseconds each.
#include <utility>

#include "device.hpp"

namespace {

using fh::fail;

constexpr int64_t kGroup = 64;
// Rows up to this run the GEMV with the norms, residual adds and SiLU fused.
constexpr int64_t kFusedRows = 8;

#define FH_TRY(call)                      \
    do {                                  \
        if (int rc_ = (call)) return rc_; \
    } while (0)

int check_weight(const char *fn, const char *what, int64_t layer, const fh_q4_weight &w, int64_t n,
                 int64_t k) {
    if (w.n != n || w.k != k)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: layer %lld %s is %lldx%lld, the config needs %lldx%lld", fn,
                    (long long)layer, what, (long long)w.n, (long long)w.k, (long long)n, (long long)k);
    return FH_OK;
}

// The model's shapes against its config, before any work is issued.
int check_model(const char *fn, const fh_llama_model &m, int64_t seq_tokens) {
    if (m.layers == nullptr && m.n_layers > 0) return fail(FH_ERR_INVALID_ARGUMENT, "%s: layers is null", fn);
    if (m.n_layers < 0 || m.hidden <= 0 || m.n_heads <= 0 || m.n_kv_heads <= 0 || m.head_dim <= 0 ||
        m.ffn <= 0 || m.vocab <= 0 || m.max_len <= 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: model sizes must be positive", fn);
    if (m.batch < 1 || m.batch > 65535)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: batch %lld is outside 1..65535", fn, (long long)m.batch);
    if (seq_tokens < 1 || seq_tokens > m.max_tokens)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: seq_tokens %lld is outside 1..max_tokens (%lld)", fn,
                    (long long)seq_tokens, (long long)m.max_tokens);
    const int64_t hq = m.n_heads * m.head_dim;
    const int64_t qkv_n = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    FH_TRY(check_weight(fn, "embed", -1, m.embed, m.vocab, m.hidden));
    for (int64_t l = 0; l < m.n_layers; ++l) {
        const fh_llama_layer &L = m.layers[l];
        FH_TRY(check_weight(fn, "qkv", l, L.qkv, qkv_n, m.hidden));
        FH_TRY(check_weight(fn, "o", l, L.o, m.hidden, hq));
        FH_TRY(check_weight(fn, "gate_up", l, L.gate_up, 2 * m.ffn, m.hidden));
        FH_TRY(check_weight(fn, "down", l, L.down, m.hidden, m.ffn));
    }
    return FH_OK;
}

int linear(fh_device *d, const uint16_t *x, int64_t rows, int64_t x_ld, const fh_q4_weight &w, uint16_t *y) {
    return fh_q4_matmul(d, x, rows, w.k, x_ld, w.wq, w.scales, w.biases, w.n, kGroup, y, FH_BF16);
}

int linear_norm(fh_device *d, const fh_llama_model &m, const uint16_t *x, const uint16_t *res, uint16_t *res_out,
                const uint16_t *weight, int64_t rows, const fh_q4_weight &w, uint16_t *y) {
    return fh_q4_matmul_rmsnorm(d, x, res, res_out, weight, m.rms_norm_eps, rows, w.k, w.wq, w.scales, w.biases,
                                w.n, kGroup, y, FH_BF16);
}

// x = rms_norm(h [+ pending]); h updated in place when pending is given.
int norm(fh_device *d, const fh_llama_model &m, int64_t rows, const uint16_t *pending, const uint16_t *weight) {
    return fh_rms_norm(d, pending ? pending : m.h, pending ? m.h : nullptr, pending ? m.h : nullptr, weight, rows,
                       m.hidden, m.rms_norm_eps, m.x);
}

// q,k = rope(q,k); cache k,v; attn = sdpa(q, cache) for every sequence.
int attention(fh_device *d, const fh_llama_model &m, const fh_llama_layer &L, int64_t seq_tokens,
              const uint32_t *positions) {
    if (seq_tokens == 1)
        return fh_decode_attention(d, m.qkv, m.batch, m.n_heads, m.n_kv_heads, m.head_dim, m.cos_tab, m.sin_tab,
                                   m.max_len, positions, L.k_cache, L.v_cache, m.max_len, m.scale,
                                   m.decode_workspace, m.decode_workspace_bytes, m.attn);
    const int64_t hq = m.n_heads * m.head_dim;
    const int64_t qkv_n = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    const int64_t seq_cache = m.n_kv_heads * m.max_len * m.head_dim;  // one sequence's cache, elements
    for (int64_t sq = 0; sq < m.batch; ++sq) {
        const int64_t r0 = sq * seq_tokens;
        uint16_t *kc = L.k_cache + sq * seq_cache, *vc = L.v_cache + sq * seq_cache;
        FH_TRY(fh_rope_kv(d, m.qkv + r0 * qkv_n, seq_tokens, m.n_heads, m.n_kv_heads, m.head_dim, m.cos_tab,
                          m.sin_tab, m.max_len, positions + r0, kc, vc, m.max_len, m.q + r0 * hq));
        FH_TRY(fh_attention(d, m.q + r0 * hq, kc, vc, positions + r0, seq_tokens, m.n_heads, m.n_kv_heads,
                            m.head_dim, m.max_len, m.scale, m.attn_workspace, m.attn_workspace_bytes,
                            m.attn + r0 * hq));
    }
    return FH_OK;
}

}  // namespace

extern "C" int fh_llama_forward(fh_device *dev, const fh_llama_model *model, int64_t seq_tokens,
                                const uint32_t *ids, const uint32_t *positions, uint32_t *next) {
    const char *fn = "fh_llama_forward";
    if (int rc = fh::check_usable(dev, fn)) return rc;
    if (model == nullptr) return fail(FH_ERR_INVALID_ARGUMENT, "%s: model is null", fn);
    const fh_llama_model &m = *model;
    FH_TRY(check_model(fn, m, seq_tokens));

    const int64_t tokens = m.batch * seq_tokens;
    const int64_t hq = m.n_heads * m.head_dim;
    FH_TRY(fh_q4_embed(dev, m.embed.wq, m.embed.scales, m.embed.biases, m.embed.n, m.embed.k, kGroup, ids, tokens,
                       m.h));
    const bool fused = tokens <= kFusedRows;
    // fused rows: the residual stream alternates between h and h2, and each
    // block's output (pending) is added inside the next RMSNorm
    uint16_t *h = m.h, *h_alt = m.h2;
    const uint16_t *pending = nullptr;
    for (int64_t l = 0; l < m.n_layers; ++l) {
        const fh_llama_layer &L = m.layers[l];
        if (!fused) {
            FH_TRY(norm(dev, m, tokens, pending, L.input_norm));
            FH_TRY(linear(dev, m.x, tokens, m.hidden, L.qkv, m.qkv));
        } else if (pending == nullptr) {
            FH_TRY(linear_norm(dev, m, h, nullptr, nullptr, L.input_norm, tokens, L.qkv, m.qkv));
        } else {
            FH_TRY(linear_norm(dev, m, pending, h, h_alt, L.input_norm, tokens, L.qkv, m.qkv));
            std::swap(h, h_alt);
        }
        FH_TRY(attention(dev, m, L, seq_tokens, positions));
        FH_TRY(linear(dev, m.attn, tokens, hq, L.o, m.o));
        if (fused) {
            // act = silu_mul(rms_norm(o + h) [Wgate; Wup]^T) in one GEMV
            const fh_q4_weight &w = L.gate_up;
            FH_TRY(fh_q4_gate_up_silu(dev, m.o, h, h_alt, L.post_norm, m.rms_norm_eps, tokens, w.k, w.wq, w.scales,
                                      w.biases, w.n, kGroup, m.act));
            std::swap(h, h_alt);
        } else {
            FH_TRY(norm(dev, m, tokens, m.o, L.post_norm));
            FH_TRY(linear(dev, m.x, tokens, m.hidden, L.gate_up, m.gate_up));
            FH_TRY(fh_silu_mul(dev, m.gate_up, tokens, m.ffn, m.act));
        }
        FH_TRY(linear(dev, m.act, tokens, m.ffn, L.down, m.o));
        pending = m.o;
    }
    // logits of each sequence's last row (src/models/llama/model.rs:112-121)
    const int64_t last = (seq_tokens - 1) * m.hidden;
    if (pending == nullptr) {
        // no layers: the embedding rows are the hidden states
        FH_TRY(norm(dev, m, tokens, nullptr, m.final_norm));
        FH_TRY(linear(dev, m.x + last, m.batch, seq_tokens * m.hidden, m.embed, m.logits));
    } else if (fused && seq_tokens == 1) {
        FH_TRY(linear_norm(dev, m, pending, h, nullptr, m.final_norm, m.batch, m.embed, m.logits));
    } else if (fused) {
        for (int64_t sq = 0; sq < m.batch; ++sq) {
            const int64_t off = sq * seq_tokens * m.hidden + last;
            FH_TRY(linear_norm(dev, m, pending + off, h + off, nullptr, m.final_norm, 1, m.embed,
                               m.logits + sq * m.vocab));
        }
    } else {
        FH_TRY(norm(dev, m, tokens, pending, m.final_norm));
        FH_TRY(linear(dev, m.x + last, m.batch, seq_tokens * m.hidden, m.embed, m.logits));
    }
    return fh_argmax(dev, m.logits, m.batch, m.vocab, next);
}

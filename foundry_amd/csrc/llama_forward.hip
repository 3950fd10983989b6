// fh_llama_forward: the decoder's layer loop, issued from native code.
//
// LlamaModel::forward (src/models/llama/model.rs:92-121) with the layer body
// of LlamaDecoderLayer::forward (:254-280), the attention of
// LlamaAttention::forward (src/models/llama/attention.rs:72-132) and the MLP
// of LlamaMlp::forward (src/models/llama/mlp.rs:49-58), then the greedy pick
// of Decoder::step (src/generate/mod.rs:192-204). Each step is one of the
// library's ops, called as a host would call it, so the results are those of
// the op-by-op sequence. One difference in how they run: above 8 rows, a
// linear whose GEMM splits K hands its f32 partials straight to the RMSNorm,
// SiLU or RoPE that consumes its output, which adds them in the order of the
// GEMM's own reduce (the same bf16 values, one launch and one round trip of
// the output fewer).
#include <utility>

#include "device.hpp"

namespace fh {
int check_q4_table(const fh_device *dev, const char *fn, const uint32_t *wq, const uint16_t *scales,
                   const uint16_t *biases, int64_t rows, int64_t k, int64_t group);
uint32_t launch_q4_gemm_deferred(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld,
                                 const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t n,
                                 uint32_t k, void *y, int y_is_f32, void *area);
void launch_rms_norm_partials(hipStream_t stream, const float *part, uint32_t splits, const uint16_t *res,
                              uint16_t *res_out, const uint16_t *w, uint32_t rows, uint32_t dim, float eps,
                              uint16_t *y);
void launch_silu_mul_partials(hipStream_t stream, const float *part, uint32_t splits, uint32_t rows, uint32_t f,
                              uint16_t *out);
bool launch_q4_gemm_direct_silu(hipStream_t stream, uint32_t cus, const uint16_t *x, uint32_t x_ld,
                                const uint32_t *wq, const uint16_t *s, const uint16_t *b, uint32_t m, uint32_t f,
                                uint32_t k, uint16_t *act);
bool attention_flash_applies(uint32_t cus, uint32_t rows, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim);
bool launch_attention_flash(hipStream_t stream, uint32_t cus, const uint16_t *q, const uint32_t *positions,
                            uint32_t rows, const uint16_t *k_cache, const uint16_t *v_cache, uint32_t n_heads,
                            uint32_t n_kv, uint32_t head_dim, uint32_t max_len, float scale, uint16_t *out,
                            uint32_t batch, uint64_t seq_cache);
int rope_kv(fh_device *dev, const char *fn, const uint16_t *qkv, const float *part, uint32_t splits,
            uint64_t part_stride, int64_t seq_tokens, int64_t n_heads, int64_t n_kv, int64_t head_dim,
            const uint16_t *cos_tab, const uint16_t *sin_tab, int64_t table_len, const uint32_t *positions,
            uint16_t *k_cache, uint16_t *v_cache, int64_t max_len, uint16_t *q_out, int64_t batch);
int q4_down_pack(fh_device *dev, const char *fn, const uint16_t *x, int64_t m, int64_t x_ld, const uint32_t *wq,
                 const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt, int64_t n,
                 int64_t k, const uint16_t *res, uint16_t *res_out, const uint16_t *norm_weight, float eps,
                 const uint32_t *next_wq, const uint16_t *next_scales, const uint16_t *next_biases,
                 const uint32_t *next_sb, const uint32_t *next_wt, int64_t next_n, bool *packed);
bool gemv_packed_applies(int64_t m, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                         const uint32_t *sb, const uint32_t *wt, int64_t n, int64_t k);
int decode_attention_with_o_image(fh_device *dev, const uint16_t *qkv, int64_t batch, int64_t n_heads, int64_t n_kv,
                                  int64_t head_dim, const uint16_t *cos_tab, const uint16_t *sin_tab,
                                  int64_t table_len, const uint32_t *positions, uint16_t *k_cache,
                                  uint16_t *v_cache, int64_t max_len, float scale, void *workspace,
                                  uint64_t workspace_bytes, uint16_t *out, bool *wrote);
int q4_gemv_packed(fh_device *dev, const char *fn, int64_t m, const uint32_t *wq, const uint16_t *scales,
                   const uint16_t *biases, const uint32_t *sb, const uint32_t *wt, int64_t n, int64_t k, void *y,
                   int y_is_f32);
int check_sb(fh_device *dev, const char *fn, const uint32_t *sb, int64_t n, int64_t k);
int check_wt(fh_device *dev, const char *fn, const uint32_t *wt, const uint32_t *sb, int64_t n, int64_t k);
int q4_matmul(fh_device *dev, const uint16_t *x, int64_t m, int64_t k, int64_t x_ld, const uint32_t *wq,
              const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt, int64_t n,
              int64_t group, void *y, int y_dtype);
int q4_matmul_rmsnorm(fh_device *dev, const uint16_t *x, const uint16_t *residual, uint16_t *residual_out,
                      const uint16_t *norm_weight, float eps, int64_t m, int64_t k, const uint32_t *wq,
                      const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt,
                      int64_t n, int64_t group, void *y, int y_dtype);
int q4_gate_up_silu(fh_device *dev, const uint16_t *x, const uint16_t *residual, uint16_t *residual_out,
                    const uint16_t *norm_weight, float eps, int64_t m, int64_t k, const uint32_t *wq,
                    const uint16_t *scales, const uint16_t *biases, const uint32_t *sb, const uint32_t *wt,
                    int64_t n, int64_t group, uint16_t *act);
}  // namespace fh

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

// Every interleaved scale/bias table and tiled word copy the model gives
// (fh_q4_weight.sb, .wt), before any work is issued: the GEMVs that read
// one get it unchecked.
int check_sb_tables(fh_device *d, const char *fn, const fh_llama_model &m) {
    FH_TRY(fh::check_sb(d, fn, m.embed.sb, m.embed.n, m.embed.k));
    FH_TRY(fh::check_wt(d, fn, m.embed.wt, m.embed.sb, m.embed.n, m.embed.k));
    for (int64_t l = 0; l < m.n_layers; ++l)
        for (const fh_q4_weight *w : {&m.layers[l].qkv, &m.layers[l].o, &m.layers[l].gate_up, &m.layers[l].down}) {
            FH_TRY(fh::check_sb(d, fn, w->sb, w->n, w->k));
            FH_TRY(fh::check_wt(d, fn, w->wt, w->sb, w->n, w->k));
            if (w->wt != nullptr && w == &m.layers[l].gate_up && w->n % 32 != 0)
                return fail(FH_ERR_INVALID_ARGUMENT, "%s: layer %lld gate_up: tiled words need n %% 32 == 0", fn,
                            (long long)l);
        }
    return FH_OK;
}

int linear(fh_device *d, const uint16_t *x, int64_t rows, int64_t x_ld, const fh_q4_weight &w, uint16_t *y) {
    return fh::q4_matmul(d, x, rows, w.k, x_ld, w.wq, w.scales, w.biases, w.sb, w.wt, w.n, kGroup, y, FH_BF16);
}

int linear_norm(fh_device *d, const fh_llama_model &m, const uint16_t *x, const uint16_t *res, uint16_t *res_out,
                const uint16_t *weight, int64_t rows, const fh_q4_weight &w, uint16_t *y) {
    return fh::q4_matmul_rmsnorm(d, x, res, res_out, weight, m.rms_norm_eps, rows, w.k, w.wq, w.scales, w.biases,
                                 w.sb, w.wt, w.n, kGroup, y, FH_BF16);
}

// x = rms_norm(h [+ pending]); h updated in place when pending is given.
int norm(fh_device *d, const fh_llama_model &m, int64_t rows, const uint16_t *pending, const uint16_t *weight) {
    return fh_rms_norm(d, pending ? pending : m.h, pending ? m.h : nullptr, pending ? m.h : nullptr, weight, rows,
                       m.hidden, m.rms_norm_eps, m.x);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The checks fh_q4_matmul makes for a GEMM of rows > 8 rows into y (bf16).
int check_gemm(fh_device *d, const char *fn, const uint16_t *x, int64_t rows, int64_t x_ld, const fh_q4_weight &w,
               const uint16_t *y) {
    FH_TRY(fh::check_q4_table(d, fn, w.wq, w.scales, w.biases, w.n, w.k, kGroup));
    if (rows > 65535ll * 128) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: m > 65535*128 rows", fn);
    if (x_ld < w.k || x_ld % 8 != 0 || x_ld > 0x7FFFFFFFll || !aligned16(x) || !aligned16(y))
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: linear operands must be 16-byte aligned with a row stride that is "
                    "a multiple of 8 and at least k", fn);
    FH_TRY(fh::check_range(d, x, (static_cast<uint64_t>(rows - 1) * x_ld + w.k) * 2, fn, "x"));
    return fh::check_range(d, y, static_cast<uint64_t>(rows) * w.n * 2, fn, "y");
}

// Runs the GEMM, leaving its K-split partials (if it splits) in the
// device's partial area for the consumer to add; returns the split count.
int gemm_deferred(fh_device *d, const char *fn, const uint16_t *x, int64_t rows, int64_t x_ld, const fh_q4_weight &w,
                  uint16_t *y, uint32_t *splits) {
    FH_TRY(fh::set_current(d, fn));
    return fh::dispatch(d, fn, [&] {
        *splits = fh::launch_q4_gemm_deferred(d->stream, d->compute_units, x, static_cast<uint32_t>(x_ld), w.wq,
                                              w.scales, w.biases, static_cast<uint32_t>(rows),
                                              static_cast<uint32_t>(w.n), static_cast<uint32_t>(w.k), y, 0,
                                              d->partial_area);
    });
}

// Above 8 rows: y = x W^T through fh_q4_matmul's checks and kernels, but
// when the GEMM splits K its partials stay in the device's partial area and
// y is not written: the op that consumes y forms each value from them in
// split order (the value the reduce would store), so the reduce launch and
// y's round trip go away and the results are those of the op sequence.
int linear_deferred(fh_device *d, const uint16_t *x, int64_t rows, int64_t x_ld, const fh_q4_weight &w, uint16_t *y,
                    uint32_t *splits) {
    const char *fn = "fh_llama_forward";
    FH_TRY(check_gemm(d, fn, x, rows, x_ld, w, y));
    return gemm_deferred(d, fn, x, rows, x_ld, w, y, splits);
}

// m.x = rms_norm(h [+ pending]), h updated when pending is given; pending is
// the output of linear_deferred with `splits` K splits.
int add_norm(fh_device *d, const fh_llama_model &m, int64_t rows, const uint16_t *pending, uint32_t splits,
             const uint16_t *norm_w) {
    if (pending == nullptr || splits <= 1) return norm(d, m, rows, pending, norm_w);
    const char *fn = "fh_llama_forward";
    const uint64_t bytes = static_cast<uint64_t>(rows) * m.hidden * 2;
    if (m.hidden % 8 != 0 || m.hidden > 8192 || !aligned16(m.h) || !aligned16(m.x) || !aligned16(norm_w))
        return fail(FH_ERR_UNSUPPORTED, "%s: the norm needs hidden %% 8 == 0, at most 8192, aligned operands", fn);
    FH_TRY(fh::check_range(d, m.h, bytes, fn, "h"));
    FH_TRY(fh::check_range(d, m.x, bytes, fn, "x"));
    FH_TRY(fh::check_range(d, norm_w, static_cast<uint64_t>(m.hidden) * 2, fn, "norm weight"));
    return fh::dispatch(d, fn, [&] {
        fh::launch_rms_norm_partials(d->stream, static_cast<const float *>(d->partial_area), splits, m.h, m.h, norm_w,
                                     static_cast<uint32_t>(rows), static_cast<uint32_t>(m.hidden), m.rms_norm_eps,
                                     m.x);
    });
}

// Above 8 rows: gate_up = m.x [Wgate; Wup]^T; act = silu(gate) * up, in the
// GEMM's epilogue where its tiles fill the chip, else the SiLU forming gate
// and up from the GEMM's output or split partials (linear_deferred).
int linear_silu(fh_device *d, const fh_llama_model &m, int64_t rows, const fh_q4_weight &w) {
    const char *fn = "fh_llama_forward";
    if (m.ffn % 8 != 0 || !aligned16(m.act)) {
        fh_q4_weight plain = w;
        plain.wt = nullptr;  // gate/up's tiled words are in the SiLU pairing, not row order
        FH_TRY(linear(d, m.x, rows, m.hidden, plain, m.gate_up));
        return fh_silu_mul(d, m.gate_up, rows, m.ffn, m.act);
    }
    FH_TRY(check_gemm(d, fn, m.x, rows, m.hidden, w, m.gate_up));
    FH_TRY(fh::check_range(d, m.act, static_cast<uint64_t>(rows) * m.ffn * 2, fn, "act"));
    // prompt-length rows whose tiles fill the chip: the activation in the
    // GEMM's epilogue (no gate/up tensor, no SiLU launch)
    bool fused = false;
    FH_TRY(fh::dispatch(d, fn, [&] {
        fused = fh::launch_q4_gemm_direct_silu(d->stream, d->compute_units, m.x, static_cast<uint32_t>(m.hidden), w.wq,
                                               w.scales, w.biases, static_cast<uint32_t>(rows),
                                               static_cast<uint32_t>(m.ffn), static_cast<uint32_t>(m.hidden), m.act);
    }));
    if (fused) return FH_OK;
    uint32_t splits = 1;
    FH_TRY(gemm_deferred(d, fn, m.x, rows, m.hidden, w, m.gate_up, &splits));
    if (splits == 1) return fh_silu_mul(d, m.gate_up, rows, m.ffn, m.act);
    return fh::dispatch(d, fn, [&] {
        fh::launch_silu_mul_partials(d->stream, static_cast<const float *>(d->partial_area), splits,
                                     static_cast<uint32_t>(rows), static_cast<uint32_t>(m.ffn), m.act);
    });
}

// q,k = rope(q,k); cache k,v; attn = sdpa(q, cache) for every sequence.
// Above one token per sequence, qkv may be the q/k/v GEMM's split partials
// (qkv_splits > 1, linear_deferred), which the RoPE then adds itself.
// One token per sequence with o_image: where the decode attention's combine
// runs it also leaves the o projection's x image in the pack area, and
// *o_image tells whether it did.
int attention(fh_device *d, const fh_llama_model &m, const fh_llama_layer &L, int64_t seq_tokens,
              const uint32_t *positions, uint32_t qkv_splits, bool *o_image = nullptr) {
    if (o_image) *o_image = false;
    if (seq_tokens == 1 && o_image)
        return fh::decode_attention_with_o_image(d, m.qkv, m.batch, m.n_heads, m.n_kv_heads, m.head_dim, m.cos_tab,
                                                 m.sin_tab, m.max_len, positions, L.k_cache, L.v_cache, m.max_len,
                                                 m.scale, m.decode_workspace, m.decode_workspace_bytes, m.attn,
                                                 o_image);
    if (seq_tokens == 1)
        return fh_decode_attention(d, m.qkv, m.batch, m.n_heads, m.n_kv_heads, m.head_dim, m.cos_tab, m.sin_tab,
                                   m.max_len, positions, L.k_cache, L.v_cache, m.max_len, m.scale,
                                   m.decode_workspace, m.decode_workspace_bytes, m.attn);
    const int64_t hq = m.n_heads * m.head_dim;
    const int64_t qkv_n = (m.n_heads + 2 * m.n_kv_heads) * m.head_dim;
    const int64_t seq_cache = m.n_kv_heads * m.max_len * m.head_dim;  // one sequence's cache, elements
    // where each sequence's call would take the one-pass kernel, the
    // sequences share one launch of it (its blocks are the per-sequence
    // launches' blocks, longest first across the batch)
    const bool one_launch =
        m.batch > 1 && m.batch <= 65535 && m.max_len <= 0xFFFFFFFFll &&
        fh::attention_flash_applies(d->compute_units, static_cast<uint32_t>(seq_tokens),
                                    static_cast<uint32_t>(m.n_heads), static_cast<uint32_t>(m.n_kv_heads),
                                    static_cast<uint32_t>(m.head_dim)) &&
        aligned16(m.q) && aligned16(m.attn) && aligned16(L.k_cache) && aligned16(L.v_cache);
    // the RoPE and cache writes of every sequence in one launch
    const float *part = qkv_splits > 1 ? static_cast<const float *>(d->partial_area) : nullptr;
    FH_TRY(fh::rope_kv(d, "fh_llama_forward", m.qkv, part, qkv_splits,
                       static_cast<uint64_t>(m.batch * seq_tokens * qkv_n), seq_tokens, m.n_heads, m.n_kv_heads,
                       m.head_dim, m.cos_tab, m.sin_tab, m.max_len, positions, L.k_cache, L.v_cache, m.max_len, m.q,
                       m.batch));
    if (!one_launch) {
        for (int64_t sq = 0; sq < m.batch; ++sq) {
            const int64_t r0 = sq * seq_tokens;
            FH_TRY(fh_attention(d, m.q + r0 * hq, L.k_cache + sq * seq_cache, L.v_cache + sq * seq_cache,
                                positions + r0, seq_tokens, m.n_heads, m.n_kv_heads, m.head_dim, m.max_len, m.scale,
                                m.attn_workspace, m.attn_workspace_bytes, m.attn + r0 * hq));
        }
        return FH_OK;
    }
    const char *fn = "fh_llama_forward";
    const uint64_t rows_bytes = static_cast<uint64_t>(m.batch) * seq_tokens * hq * 2;
    const uint64_t cache_bytes = static_cast<uint64_t>(m.batch) * seq_cache * 2;
    FH_TRY(fh::check_range(d, m.q, rows_bytes, fn, "q"));
    FH_TRY(fh::check_range(d, m.attn, rows_bytes, fn, "attn"));
    FH_TRY(fh::check_range(d, L.k_cache, cache_bytes, fn, "k_cache"));
    FH_TRY(fh::check_range(d, L.v_cache, cache_bytes, fn, "v_cache"));
    FH_TRY(fh::check_range(d, positions, static_cast<uint64_t>(m.batch) * seq_tokens * 4, fn, "positions"));
    return fh::dispatch(d, fn, [&] {
        fh::launch_attention_flash(d->stream, d->compute_units, m.q, positions, static_cast<uint32_t>(seq_tokens),
                                   L.k_cache, L.v_cache, static_cast<uint32_t>(m.n_heads),
                                   static_cast<uint32_t>(m.n_kv_heads), static_cast<uint32_t>(m.head_dim),
                                   static_cast<uint32_t>(m.max_len), m.scale, m.attn, static_cast<uint32_t>(m.batch),
                                   static_cast<uint64_t>(seq_cache));
    });
}

}  // namespace

extern "C" int fh_llama_forward(fh_device *dev, const fh_llama_model *model, int64_t seq_tokens,
                                const uint32_t *ids, const uint32_t *positions, uint32_t *next) {
    const char *fn = "fh_llama_forward";
    if (int rc = fh::check_usable(dev, fn)) return rc;
    if (model == nullptr) return fail(FH_ERR_INVALID_ARGUMENT, "%s: model is null", fn);
    const fh_llama_model &m = *model;
    FH_TRY(check_model(fn, m, seq_tokens));
    FH_TRY(check_sb_tables(dev, fn, m));

    const int64_t tokens = m.batch * seq_tokens;
    const int64_t hq = m.n_heads * m.head_dim;
    FH_TRY(fh_q4_embed(dev, m.embed.wq, m.embed.scales, m.embed.biases, m.embed.n, m.embed.k, kGroup, ids, tokens,
                       m.h));
    const bool fused = tokens <= kFusedRows;
    // fused rows: the residual stream alternates between h and h2, and each
    // block's output (pending) is added inside the next RMSNorm
    uint16_t *h = m.h, *h_alt = m.h2;
    const uint16_t *pending = nullptr;
    uint32_t pending_splits = 1;  // above 8 rows: K splits of the GEMM behind pending
    // batched decode: the down projection left the next RMSNorm'd GEMV's
    // image in the pack area (q4_down_pack) and h_alt = pending + h
    bool packed = false;
    for (int64_t l = 0; l < m.n_layers; ++l) {
        const fh_llama_layer &L = m.layers[l];
        uint32_t qkv_splits = 1;
        if (packed) {
            FH_TRY(fh::q4_gemv_packed(dev, fn, tokens, L.qkv.wq, L.qkv.scales, L.qkv.biases, L.qkv.sb, L.qkv.wt,
                                      L.qkv.n, L.qkv.k, m.qkv, 0));
            std::swap(h, h_alt);
        } else if (!fused) {
            FH_TRY(add_norm(dev, m, tokens, pending, pending_splits, L.input_norm));
            // one token per sequence: fh_decode_attention reads qkv itself
            if (seq_tokens > 1)
                FH_TRY(linear_deferred(dev, m.x, tokens, m.hidden, L.qkv, m.qkv, &qkv_splits));
            else
                FH_TRY(linear(dev, m.x, tokens, m.hidden, L.qkv, m.qkv));
        } else if (pending == nullptr) {
            FH_TRY(linear_norm(dev, m, h, nullptr, nullptr, L.input_norm, tokens, L.qkv, m.qkv));
        } else {
            FH_TRY(linear_norm(dev, m, pending, h, h_alt, L.input_norm, tokens, L.qkv, m.qkv));
            std::swap(h, h_alt);
        }
        // the batched decode step: the o projection can read its x as the
        // image the attention's combine leaves in the pack area
        bool o_image = false;
        const bool want_o_image = fused && seq_tokens == 1 &&
                                  fh::gemv_packed_applies(tokens, L.o.wq, L.o.scales, L.o.biases, L.o.sb, L.o.wt,
                                                          L.o.n, L.o.k);
        FH_TRY(attention(dev, m, L, seq_tokens, positions, qkv_splits, want_o_image ? &o_image : nullptr));
        if (!fused) {
            // o, then h += o and x = rms_norm(h); gate/up and SiLU; down (its
            // output is added by the next RMSNorm)
            uint32_t o_splits = 1;
            FH_TRY(linear_deferred(dev, m.attn, tokens, hq, L.o, m.o, &o_splits));
            FH_TRY(add_norm(dev, m, tokens, m.o, o_splits, L.post_norm));
            FH_TRY(linear_silu(dev, m, tokens, L.gate_up));
            FH_TRY(linear_deferred(dev, m.act, tokens, m.ffn, L.down, m.o, &pending_splits));
            pending = m.o;
            continue;
        }
        if (o_image)
            FH_TRY(fh::q4_gemv_packed(dev, fn, tokens, L.o.wq, L.o.scales, L.o.biases, L.o.sb, L.o.wt, L.o.n, L.o.k,
                                      m.o, 0));
        else
            FH_TRY(linear(dev, m.attn, tokens, hq, L.o, m.o));
        {
            // act = silu_mul(rms_norm(o + h) [Wgate; Wup]^T) in one GEMV
            const fh_q4_weight &w = L.gate_up;
            FH_TRY(fh::q4_gate_up_silu(dev, m.o, h, h_alt, L.post_norm, m.rms_norm_eps, tokens, w.k, w.wq,
                                       w.scales, w.biases, w.sb, w.wt, w.n, kGroup, m.act));
            std::swap(h, h_alt);
        }
        packed = false;
        if (seq_tokens == 1) {
            // the next RMSNorm'd GEMV: the next layer's q/k/v, or the LM head
            const bool last = l + 1 == m.n_layers;
            const fh_q4_weight &nw = last ? m.embed : m.layers[l + 1].qkv;
            const uint16_t *norm_w = last ? m.final_norm : m.layers[l + 1].input_norm;
            const fh_q4_weight &w = L.down;
            FH_TRY(fh::q4_down_pack(dev, fn, m.act, tokens, m.ffn, w.wq, w.scales, w.biases, w.sb, w.wt, w.n, w.k,
                                    h, last ? nullptr : h_alt, norm_w, m.rms_norm_eps, nw.wq, nw.scales, nw.biases,
                                    nw.sb, nw.wt, nw.n, &packed));
        }
        if (!packed) FH_TRY(linear(dev, m.act, tokens, m.ffn, L.down, m.o));
        pending = m.o;
    }
    // logits of each sequence's last row (src/models/llama/model.rs:112-121)
    const int64_t last = (seq_tokens - 1) * m.hidden;
    if (pending == nullptr) {
        // no layers: the embedding rows are the hidden states
        FH_TRY(norm(dev, m, tokens, nullptr, m.final_norm));
        FH_TRY(linear(dev, m.x + last, m.batch, seq_tokens * m.hidden, m.embed, m.logits));
    } else if (packed) {
        FH_TRY(fh::q4_gemv_packed(dev, fn, m.batch, m.embed.wq, m.embed.scales, m.embed.biases, m.embed.sb,
                                  m.embed.wt, m.embed.n, m.embed.k, m.logits, 0));
    } else if (fused && seq_tokens == 1) {
        FH_TRY(linear_norm(dev, m, pending, h, nullptr, m.final_norm, m.batch, m.embed, m.logits));
    } else if (fused) {
        for (int64_t sq = 0; sq < m.batch; ++sq) {
            const int64_t off = sq * seq_tokens * m.hidden + last;
            FH_TRY(linear_norm(dev, m, pending + off, h + off, nullptr, m.final_norm, 1, m.embed,
                               m.logits + sq * m.vocab));
        }
    } else {
        FH_TRY(add_norm(dev, m, tokens, pending, pending_splits, m.final_norm));
        FH_TRY(linear(dev, m.x + last, m.batch, seq_tokens * m.hidden, m.embed, m.logits));
    }
    return fh_argmax(dev, m.logits, m.batch, m.vocab, next);
}

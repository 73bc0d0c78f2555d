// .aidn checkpoints (AidenModel, aideen-core/src/model.rs:10-58).  The reference writes them with
// bincode 1.3 under its default options: little-endian fixed-width integers, a u64 length before
// every string and sequence, bool as one byte, struct fields in declaration order, maps as a u64
// entry count followed by key/value pairs (in the writer's hash order).  The file is
//   AidenModel { config: ArchitectureConfig, weights: HashMap<String, Vec<f32>>,
//                metadata: HashMap<String, String> }
// with ArchitectureConfig as declared in aideen-core/src/state.rs:7-35 (usize fields are u64).
//
// adn_aidn_weights maps the reference's names and layouts onto adn_weights:
//   FixedPointMemoryReasoning::export_weights (fixed_point_memory_reasoning.rs:626-784): one shared
//     row-major [d][d] matrix each for w_q, w_k, w_v, w_o, w_in, w_x, w_out, w_hist_shared (the
//     CPU model shares them over the slots), [H][d] q_bias, k_bias, slot_anchor, a_log,
//     hist_slot_scale, [d] norm_scale and b_delta, [H] hist_gate_logit, [(H d)][r] w_k_write,
//     [(H r)][d] w_v_write, and the scalar damping;
//   LmHead::export_weights (lm_head.rs:169-188): head.w [V][d] row-major, head.b [V], head.g [d];
//   Trainer::save_full (trainer.rs:6515-6520): tokenizer.embeddings, nalgebra's column-major
//     storage of the [V][d] table, i.e. [d][V].
// Shared matrices are replicated per slot (the per-slot engine with equal slots computes the
// shared-weight model), the embedding is transposed to [V][d], and the carrier takes W_x's
// diagonal (temporal_step, fixed_point_memory_reasoning.rs:1471-1475).
#include <algorithm>
#include <cerrno>
#include <climits>
#include <cstdio>
#include <memory>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "aideen_hip.h"

namespace adn {
void set_error(const std::string &msg);
}

struct adn_aidn {
    adn_aidn_config cfg{};
    std::vector<std::string> names;                       // weight names in file order
    std::unordered_map<std::string, std::vector<float>> weights;
    std::vector<std::string> meta_keys;
    std::unordered_map<std::string, std::string> meta;
    // arrays handed out by adn_aidn_weights (live until adn_aidn_close)
    std::unordered_map<std::string, std::vector<float>> prepared;
};

namespace {

struct Reader {
    FILE *f;
    long long left;  // bytes not yet read
    std::string err;
    bool take(void *dst, long long n) {
        if (!err.empty()) return false;
        if (n < 0 || n > left) {
            err = "truncated or corrupt .aidn file";
            return false;
        }
        if (n && fread(dst, 1, (size_t)n, f) != (size_t)n) {
            err = "read error";
            return false;
        }
        left -= n;
        return true;
    }
    bool u64(uint64_t &v) { return take(&v, 8); }
    bool usize(int64_t &v) {
        uint64_t x = 0;
        if (!u64(x)) return false;
        if (x > (uint64_t)INT64_MAX) {
            err = "integer out of range";
            return false;
        }
        v = (int64_t)x;
        return true;
    }
    bool f32(float &v) { return take(&v, 4); }
    bool boolean(int32_t &v) {
        uint8_t b = 0;
        if (!take(&b, 1)) return false;
        if (b > 1) {
            err = "invalid bool";
            return false;
        }
        v = b;
        return true;
    }
    bool str(std::string &s) {
        uint64_t n = 0;
        if (!u64(n)) return false;
        if ((long long)n < 0 || (long long)n > left) {
            err = "truncated or corrupt .aidn file";
            return false;
        }
        s.resize((size_t)n);
        return take(&s[0], (long long)n);
    }
    bool floats(std::vector<float> &v) {
        uint64_t n = 0;
        if (!u64(n)) return false;
        if (n > (uint64_t)(left / 4)) {
            err = "truncated or corrupt .aidn file";
            return false;
        }
        v.resize((size_t)n);
        return take(v.data(), (long long)n * 4);
    }
};

int fail_invalid(const std::string &msg) {
    adn::set_error(msg);
    return ADN_E_INVALID;
}

}  // namespace

extern "C" {

static int aidn_open(const char *path, adn_aidn **out);
static int aidn_weights(adn_aidn *m, adn_weights *w, adn_config *cfg, adn_run *run);

// No C++ exception (an allocation failure on a corrupt file's sizes) crosses the C ABI.
int adn_aidn_open(const char *path, adn_aidn **out) {
    try {
        return aidn_open(path, out);
    } catch (const std::exception &e) {
        return fail_invalid(std::string("cannot load .aidn file: ") + e.what());
    }
}

int adn_aidn_weights(adn_aidn *m, adn_weights *w, adn_config *cfg, adn_run *run) {
    try {
        return aidn_weights(m, w, cfg, run);
    } catch (const std::exception &e) {
        return fail_invalid(std::string("cannot map .aidn weights: ") + e.what());
    }
}

static int aidn_open(const char *path, adn_aidn **out) {
    if (!path || !out) return fail_invalid("null argument");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) return fail_invalid(std::string("cannot open ") + path);
    fseek(f, 0, SEEK_END);
    const long long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    Reader r{f, size, {}};
    struct Closer {  // the file is closed on every path, an exception's included
        FILE *&f;
        ~Closer() {
            if (f) fclose(f);
        }
    } closer{f};
    std::unique_ptr<adn_aidn> owner(new adn_aidn());
    adn_aidn *m = owner.get();
    adn_aidn_config &c = m->cfg;
    r.usize(c.d_m) && r.usize(c.d_r) && r.usize(c.d_c) && r.usize(c.d_e) && r.usize(c.d_sim) &&
        r.usize(c.h_slots) && r.usize(c.vocab_size) && r.usize(c.ctx_len) && r.usize(c.max_deq_iters) &&
        r.f32(c.deq_epsilon) && r.usize(c.adj_iters) && r.boolean(c.train_deq) && r.f32(c.deq_grad_scale) &&
        r.usize(c.renorm_every_steps) && r.usize(c.num_samples) && r.f32(c.weight_decay);
    uint64_t nw = 0;
    if (r.u64(nw)) {
        for (uint64_t i = 0; i < nw && r.err.empty(); ++i) {
            std::string name;
            std::vector<float> v;
            if (!r.str(name) || !r.floats(v)) break;
            if (!m->weights.count(name)) m->names.push_back(name);
            m->weights[name] = std::move(v);
        }
    }
    uint64_t nm = 0;
    if (r.err.empty() && r.u64(nm)) {
        for (uint64_t i = 0; i < nm && r.err.empty(); ++i) {
            std::string k, v;
            if (!r.str(k) || !r.str(v)) break;
            if (!m->meta.count(k)) m->meta_keys.push_back(k);
            m->meta[k] = v;
        }
    }
    if (!r.err.empty()) return fail_invalid(r.err + " (" + path + ")");
    if (r.left != 0) return fail_invalid(std::string("trailing bytes after the model (") + path + ")");
    *out = owner.release();
    return ADN_OK;
}

void adn_aidn_close(adn_aidn *m) { delete m; }

int adn_aidn_config_get(const adn_aidn *m, adn_aidn_config *out) {
    if (!m || !out) return fail_invalid("null argument");
    *out = m->cfg;
    return ADN_OK;
}

int adn_aidn_count(const adn_aidn *m, int32_t *n_weights, int32_t *n_metadata) {
    if (!m) return fail_invalid("null argument");
    if (n_weights) *n_weights = (int32_t)m->names.size();
    if (n_metadata) *n_metadata = (int32_t)m->meta_keys.size();
    return ADN_OK;
}

int adn_aidn_name(const adn_aidn *m, int32_t i, const char **name) {
    if (!m || !name) return fail_invalid("null argument");
    if (i < 0 || i >= (int32_t)m->names.size()) return fail_invalid("weight index out of range");
    *name = m->names[(size_t)i].c_str();
    return ADN_OK;
}

int adn_aidn_tensor(const adn_aidn *m, const char *name, const float **data, int64_t *count) {
    if (!m || !name || !data || !count) return fail_invalid("null argument");
    auto it = m->weights.find(name);
    *data = it == m->weights.end() ? nullptr : it->second.data();
    *count = it == m->weights.end() ? 0 : (int64_t)it->second.size();
    return ADN_OK;
}

int adn_aidn_metadata(const adn_aidn *m, const char *key, const char **value) {
    if (!m || !key || !value) return fail_invalid("null argument");
    auto it = m->meta.find(key);
    *value = it == m->meta.end() ? nullptr : it->second.c_str();
    return ADN_OK;
}

static int aidn_weights(adn_aidn *m, adn_weights *w, adn_config *cfg, adn_run *run) {
    if (!m || !w) return fail_invalid("null argument");
    const int64_t d = m->cfg.d_r, H = m->cfg.h_slots;
    int64_t V = m->cfg.vocab_size;
    auto mv = m->meta.find("vocab_size");  // the trainer sizes the tokenizer from the metadata
    if (mv != m->meta.end()) {
        const char *txt = mv->second.c_str();
        char *end = nullptr;
        errno = 0;
        const long long v = std::strtoll(txt, &end, 10);
        if (errno || end == txt || *end != '\0') return fail_invalid("metadata vocab_size is not an integer");
        V = v;
    }
    constexpr int64_t R = 32;  // RETAIN_RANK (fixed_point_memory_reasoning.rs:291)
    // Bounds before any size product: with these, every tensor size below fits comfortably in
    // 64 bits (V * d < 2^42) and the int32 fields of adn_config cannot truncate.
    if (d < 1 || d > 2048) return fail_invalid("model d_r outside [1, 2048]");
    if (H < 1 || H > 16) return fail_invalid("model h_slots outside [1, 16]");
    if (V < 1 || V > INT32_MAX) return fail_invalid("model vocab_size outside [1, 2^31)");
    std::string err;
    auto get = [&](const char *name, int64_t n, bool required) -> const std::vector<float> * {
        auto it = m->weights.find(name);
        if (it == m->weights.end()) {
            if (required && err.empty()) err = std::string("weight ") + name + " not found";
            return nullptr;
        }
        if ((int64_t)it->second.size() != n) {
            if (err.empty())
                err = std::string("weight ") + name + " size mismatch: expected " + std::to_string(n) + ", got " +
                      std::to_string(it->second.size());
            return nullptr;
        }
        return &it->second;
    };
    const auto *wq = get("reasoning.w_q", d * d, true), *wk = get("reasoning.w_k", d * d, true);
    const auto *wv = get("reasoning.w_v", d * d, true), *wo = get("reasoning.w_o", d * d, true);
    const auto *win = get("reasoning.w_in", d * d, true), *wx = get("reasoning.w_x", d * d, true);
    const auto *wout = get("reasoning.w_out", d * d, true), *alog = get("reasoning.a_log", H * d, true);
    const auto *ns = get("reasoning.norm_scale", d, true);
    const auto *anchor = get("reasoning.slot_anchor", H * d, false);
    const auto *qb = get("reasoning.q_bias", H * d, false), *kb = get("reasoning.k_bias", H * d, false);
    const auto *whist = get("reasoning.w_hist_shared", d * d, false);
    const auto *hscale = get("reasoning.hist_slot_scale", H * d, false);
    const auto *hgate = get("reasoning.hist_gate_logit", H, false);
    const auto *bdelta = get("reasoning.b_delta", d, false);
    const auto *wkw = get("reasoning.w_k_write", H * d * R, false);
    const auto *wvw = get("reasoning.w_v_write", H * R * d, false);
    const auto *damp = get("reasoning.damping", 1, false);
    const auto *emb = get("tokenizer.embeddings", V * d, true);
    const auto *hw = get("head.w", V * d, true), *hb = get("head.b", V, true), *hg = get("head.g", d, true);
    if (err.empty() && !anchor)  // the reference falls back to a seeded random draw (StdRng), not reproducible here
        err = "weight reasoning.slot_anchor not found (its fallback is the reference's seeded random draw)";
    if (!err.empty()) return fail_invalid(err);

    auto &P = m->prepared;
    P.clear();
    auto per_slot = [&](const char *key, const std::vector<float> &src) -> const float * {
        std::vector<float> &v = P[key];
        v.resize((size_t)(H * (int64_t)src.size()));
        for (int64_t s = 0; s < H; ++s) std::memcpy(&v[(size_t)(s * (int64_t)src.size())], src.data(), src.size() * 4);
        return v.data();
    };
    std::memset(w, 0, sizeof(*w));
    w->w_q = per_slot("w_q", *wq);
    w->w_k = per_slot("w_k", *wk);
    w->w_v = per_slot("w_v", *wv);
    w->w_o = per_slot("w_o", *wo);
    w->w_in = per_slot("w_in", *win);
    w->w_out = per_slot("w_out", *wout);
    {
        std::vector<float> &v = P["wx_diag"];
        v.resize((size_t)(H * d));
        for (int64_t s = 0; s < H; ++s)
            for (int64_t i = 0; i < d; ++i) v[(size_t)(s * d + i)] = (*wx)[(size_t)(i * d + i)];
        w->wx_diag = v.data();
    }
    {
        std::vector<float> &v = P["embed"];
        v.resize((size_t)(V * d));
        const std::vector<float> &e = *emb;  // column-major [d][V], transposed in 64x64 tiles
        constexpr int64_t TB = 64;
        for (int64_t j0 = 0; j0 < d; j0 += TB)
            for (int64_t i0 = 0; i0 < V; i0 += TB) {
                const int64_t j1 = std::min(d, j0 + TB), i1 = std::min(V, i0 + TB);
                for (int64_t i = i0; i < i1; ++i)
                    for (int64_t j = j0; j < j1; ++j) v[(size_t)(i * d + j)] = e[(size_t)(j * V + i)];
            }
        w->embed = v.data();
    }
    w->q_bias = qb ? qb->data() : nullptr;
    w->k_bias = kb ? kb->data() : nullptr;
    w->anchor = anchor->data();
    w->norm_scale = ns->data();
    w->lm_w = hw->data();
    w->lm_b = hb->data();
    w->lm_g = hg->data();
    w->a_log = alog->data();
    w->b_delta = bdelta ? per_slot("b_delta", *bdelta) : nullptr;
    w->w_kw = wkw ? wkw->data() : nullptr;
    w->w_vw = wvw ? wvw->data() : nullptr;
    w->w_hist = whist ? whist->data() : nullptr;
    w->hist_slot_scale = hscale ? hscale->data() : nullptr;
    w->hist_gate_logit = hgate ? hgate->data() : nullptr;
    if (cfg) {
        std::memset(cfg, 0, sizeof(*cfg));
        cfg->d_r = (int32_t)d;
        cfg->h_slots = (int32_t)H;
        cfg->vocab = (int32_t)V;
        cfg->d_state = 1;
        cfg->rank = (int32_t)R;
        cfg->max_batch = 1;
        cfg->max_seq = (int32_t)std::max<int64_t>(1, std::min<int64_t>(m->cfg.ctx_len, 1 << 24));
        cfg->anderson_m = 0;
        cfg->flags = 0;
    }
    if (run) {
        std::memset(run, 0, sizeof(*run));
        run->batch = 1;
        run->seq = 1;
        run->max_iters = (int32_t)std::max<int64_t>(1, std::min<int64_t>(m->cfg.max_deq_iters, 256));
        run->eps = m->cfg.deq_epsilon;
        run->damping = damp ? (*damp)[0] : 0.70f;  // FixedPointMemoryReasoning's default (:458)
    }
    return ADN_OK;
}

}  // extern "C"

// Host feed of the training step: the packed token stream with sliding
// windows (train/dataset.zig) and the fine-tune loop around Runner.step
// (commands/finetune.zig).  Host code only; the loop drives the Runner
// through its public C ABI.
#include <ctype.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <string>
#include <vector>

#include "internal.hpp"

using namespace vkh;

struct vkh_dataset {
    std::vector<uint32_t> packed;
    uint32_t n_pos = 0;
    size_t num_batches() const { return packed.size() <= n_pos ? 0 : packed.size() - n_pos; }
};

namespace {

// ── a small JSON reader: enough to find an integer array field ──────────
// Values are parsed fully (objects, arrays, strings with escapes, numbers,
// literals) so malformed lines are rejected as a whole, as a JSON parser
// would; only the "ids" member's value is kept.
struct Json {
    const char *p, *end;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\r' || *p == '\n')) ++p;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n)) return false;
        p += n;
        return true;
    }
    bool string(std::string *out) {
        if (p >= end || *p != '"') return false;
        ++p;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) return false;
                const char e = *p;
                if (e == 'u') {
                    if (end - p < 5) return false;
                    for (int i = 1; i <= 4; ++i)
                        if (!isxdigit((unsigned char)p[i])) return false;
                    p += 4;
                } else if (!strchr("\"\\/bfnrt", e)) {
                    return false;
                }
                if (out) out->push_back('?');
            } else {
                if ((unsigned char)*p < 0x20) return false;
                if (out) out->push_back(*p);
            }
            ++p;
        }
        if (p >= end) return false;
        ++p;
        return true;
    }
    // number; *is_u32 / *val report a non-negative integer below 2^32
    bool number(bool *is_u32, uint64_t *val) {
        const char *s = p;
        if (p < end && *p == '-') ++p;
        if (p >= end || !isdigit((unsigned char)*p)) return false;
        if (*p == '0') ++p;
        else while (p < end && isdigit((unsigned char)*p)) ++p;
        bool integral = true;
        if (p < end && *p == '.') {
            integral = false;
            ++p;
            if (p >= end || !isdigit((unsigned char)*p)) return false;
            while (p < end && isdigit((unsigned char)*p)) ++p;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            if (p >= end || !isdigit((unsigned char)*p)) return false;
            while (p < end && isdigit((unsigned char)*p)) ++p;
        }
        *is_u32 = false;
        if (integral && *s != '-' && p - s <= 10) {
            uint64_t v = 0;
            for (const char *q = s; q < p; ++q) v = v * 10 + (uint64_t)(*q - '0');
            if (v <= 0xffffffffull) {
                *is_u32 = true;
                *val = v;
            }
        }
        return true;
    }
    // value; when ids != nullptr and the value is an array of u32 integers,
    // they are appended and *ids_ok is set
    bool value(std::vector<uint32_t> *ids, bool *ids_ok, int depth) {
        if (depth > 64) return false;
        ws();
        if (p >= end) return false;
        if (*p == '{') return object(nullptr, nullptr, depth + 1);
        if (*p == '[') {
            ++p;
            bool all_int = true;
            std::vector<uint32_t> tmp;
            ws();
            if (p < end && *p == ']') {
                ++p;
            } else {
                for (;;) {
                    ws();
                    if (p < end && (isdigit((unsigned char)*p) || *p == '-')) {
                        bool u = false;
                        uint64_t v = 0;
                        if (!number(&u, &v)) return false;
                        if (u) tmp.push_back((uint32_t)v);
                        else all_int = false;
                    } else {
                        all_int = false;
                        if (!value(nullptr, nullptr, depth + 1)) return false;
                    }
                    ws();
                    if (p < end && *p == ',') { ++p; continue; }
                    if (p < end && *p == ']') { ++p; break; }
                    return false;
                }
            }
            if (ids && all_int) {
                *ids = std::move(tmp);
                *ids_ok = true;
            }
            return true;
        }
        if (*p == '"') return string(nullptr);
        if (*p == 't') return lit("true");
        if (*p == 'f') return lit("false");
        if (*p == 'n') return lit("null");
        bool u = false;
        uint64_t v = 0;
        return number(&u, &v);
    }
    // object; the top-level call collects the "ids" member
    bool object(std::vector<uint32_t> *ids, bool *ids_ok, int depth) {
        if (p >= end || *p != '{') return false;
        ++p;
        ws();
        if (p < end && *p == '}') { ++p; return true; }
        for (;;) {
            ws();
            std::string key;
            if (!string(&key)) return false;
            ws();
            if (p >= end || *p != ':') return false;
            ++p;
            const bool want = ids && key == "ids";
            if (want) *ids_ok = false;  // a later duplicate key decides, as in a map
            if (!value(want ? ids : nullptr, want ? ids_ok : nullptr, depth)) return false;
            ws();
            if (p < end && *p == ',') { ++p; continue; }
            if (p < end && *p == '}') { ++p; return true; }
            return false;
        }
    }
};

// One JSONL line -> token ids, or false when the line is to be skipped.
bool parse_line(const char *b, const char *e, std::vector<uint32_t> &ids) {
    Json j{b, e};
    j.ws();
    if (j.p >= j.end || *j.p != '{') return false;
    bool ok = false;
    if (!j.object(&ids, &ok, 0)) return false;
    j.ws();
    return j.p == j.end && ok;
}

vkh_status check_dataset(const vkh_dataset *d) {
    if (!d) return fail(VKH_ERR_INVALID_ARGUMENT, "null dataset");
    return VKH_OK;
}

}  // namespace

extern "C" {

vkh_status vkh_dataset_from_examples(const uint32_t *const *examples, const size_t *lens,
                                     size_t n_examples, uint32_t n_pos, uint32_t eos_id,
                                     vkh_dataset **out) {
    if (!out || (n_examples && (!examples || !lens)))
        return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    vkh_dataset *d = new vkh_dataset;
    d->n_pos = n_pos;
    for (size_t i = 0; i < n_examples; ++i) {
        if (lens[i] && !examples[i]) {
            delete d;
            return fail(VKH_ERR_INVALID_ARGUMENT, "example %zu is null", i);
        }
        if (lens[i]) d->packed.insert(d->packed.end(), examples[i], examples[i] + lens[i]);
        if (i + 1 < n_examples) d->packed.push_back(eos_id);  // dataset.zig:91
    }
    *out = d;
    return VKH_OK;
}

vkh_status vkh_dataset_from_jsonl(const char *path, uint32_t n_pos, uint32_t eos_id,
                                  vkh_dataset **out) {
    if (!path || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) return fail(VKH_ERR_IO, "cannot open %s", path);
    std::string buf;
    char chunk[1 << 16];
    size_t n;
    while ((n = fread(chunk, 1, sizeof chunk, f)) > 0) buf.append(chunk, n);
    const bool err = ferror(f);
    fclose(f);
    if (err) return fail(VKH_ERR_IO, "read error on %s", path);

    vkh_dataset *d = new vkh_dataset;
    d->n_pos = n_pos;
    size_t lines = 0;
    std::vector<uint32_t> ids;
    const char *p = buf.data(), *end = buf.data() + buf.size();
    while (p <= end) {
        const char *nl = (const char *)memchr(p, '\n', (size_t)(end - p));
        const char *le = nl ? nl : end;
        // trim " \t\r" (dataset.zig:120)
        const char *b = p, *e = le;
        while (b < e && (*b == ' ' || *b == '\t' || *b == '\r')) ++b;
        while (e > b && (e[-1] == ' ' || e[-1] == '\t' || e[-1] == '\r')) --e;
        if (b < e) {
            ids.clear();
            if (parse_line(b, e, ids)) {
                if (lines > 0) d->packed.push_back(eos_id);  // dataset.zig:134
                d->packed.insert(d->packed.end(), ids.begin(), ids.end());
                ++lines;
            }
        }
        if (!nl) break;
        p = nl + 1;
    }
    if (lines == 0) {
        delete d;
        return fail(VKH_ERR_EMPTY_DATASET, "no usable line in %s", path);
    }
    *out = d;
    return VKH_OK;
}

void vkh_dataset_destroy(vkh_dataset *d) { delete d; }

size_t vkh_dataset_num_batches(const vkh_dataset *d) { return d ? d->num_batches() : 0; }

size_t vkh_dataset_packed_len(const vkh_dataset *d) { return d ? d->packed.size() : 0; }

vkh_status vkh_dataset_packed(const vkh_dataset *d, uint32_t *out, size_t n) {
    VKH_TRY(check_dataset(d));
    if (!out || n != d->packed.size())
        return fail(VKH_ERR_INVALID_ARGUMENT, "output length %zu != %zu", n, d->packed.size());
    memcpy(out, d->packed.data(), n * 4);
    return VKH_OK;
}

vkh_status vkh_dataset_batch(const vkh_dataset *d, size_t idx, uint32_t *input_ids, size_t n_input,
                             uint32_t *target_ids, size_t n_target) {
    VKH_TRY(check_dataset(d));
    if (n_input != d->n_pos) return fail(VKH_ERR_INPUT_IDS_LEN, "input_ids len %zu != %u", n_input, d->n_pos);
    if (n_target != d->n_pos)
        return fail(VKH_ERR_TARGET_IDS_LEN, "target_ids len %zu != %u", n_target, d->n_pos);
    if (idx >= d->num_batches())
        return fail(VKH_ERR_BATCH_INDEX_OUT_OF_RANGE, "batch %zu of %zu", idx, d->num_batches());
    if (d->n_pos && (!input_ids || !target_ids)) return fail(VKH_ERR_INVALID_ARGUMENT, "null output");
    memcpy(input_ids, d->packed.data() + idx, (size_t)d->n_pos * 4);
    memcpy(target_ids, d->packed.data() + idx + 1, (size_t)d->n_pos * 4);
    return VKH_OK;
}

vkh_status vkh_dataset_batch_seqs(const vkh_dataset *d, size_t idx, size_t stride, uint32_t n_seqs,
                                  uint32_t *input_ids, uint32_t *target_ids) {
    VKH_TRY(check_dataset(d));
    const size_t nb = d->num_batches();
    if (nb == 0 || idx >= nb)
        return fail(VKH_ERR_BATCH_INDEX_OUT_OF_RANGE, "batch %zu of %zu", idx, nb);
    for (uint32_t s = 0; s < n_seqs; ++s) {
        const size_t w = (idx + (size_t)s * stride) % nb;
        VKH_TRY(vkh_dataset_batch(d, w, input_ids + (size_t)s * d->n_pos, d->n_pos,
                                  target_ids + (size_t)s * d->n_pos, d->n_pos));
    }
    return VKH_OK;
}

float vkh_mean_ce(const float *logits, const uint32_t *target_ids, size_t n_rows, size_t vocab) {
    if (!logits || !target_ids || n_rows == 0 || vocab == 0) return NAN;
    double ce_sum = 0;
    for (size_t r = 0; r < n_rows; ++r) {
        const float *row = logits + r * vocab;
        float m = -INFINITY;
        for (size_t o = 0; o < vocab; ++o) m = fmaxf(m, row[o]);
        double sum_e = 0;
        for (size_t o = 0; o < vocab; ++o) sum_e += exp((double)row[o] - (double)m);
        const double log_z = (double)m + log(sum_e);
        const uint32_t t = target_ids[r];
        ce_sum += log_z - (t < vocab ? (double)row[t] : NAN);
    }
    return (float)(ce_sum / (double)n_rows);
}

vkh_status vkh_runner_finetune(vkh_runner *r, const vkh_dataset *d, uint32_t batch_idx,
                               uint32_t n_steps, uint32_t rotate, vkh_finetune_result *out) {
    if (!r || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    VKH_TRY(check_dataset(d));
    vkh_config cfg;
    VKH_TRY(vkh_runner_get_config(r, &cfg));
    if (cfg.n_pos != d->n_pos)
        return fail(VKH_ERR_INVALID_ARGUMENT, "dataset n_pos %u != runner n_pos %u", d->n_pos, cfg.n_pos);
    const size_t nb = d->num_batches();
    if (nb == 0) return fail(VKH_ERR_DATASET_TOO_SHORT, "dataset has no batch at n_pos %u", d->n_pos);
    if (batch_idx >= nb) return fail(VKH_ERR_BATCH_IDX_OUT_OF_RANGE, "batch %u of %zu", batch_idx, nb);
    const uint32_t seqs = cfg.n_seqs ? cfg.n_seqs : 1;
    const size_t T = (size_t)seqs * cfg.n_pos, V = cfg.vocab_size;
    std::vector<uint32_t> in(T), tg(T);
    std::vector<float> logits;
    auto ce_on = [&](float *ce) -> vkh_status {
        VKH_TRY(vkh_dataset_batch_seqs(d, batch_idx, cfg.n_pos, seqs, in.data(), tg.data()));
        logits.resize(T * V);
        VKH_TRY(vkh_runner_forward_logits(r, in.data(), T, logits.data(), logits.size()));
        *ce = vkh_mean_ce(logits.data(), tg.data(), T, V);
        return VKH_OK;
    };
    VKH_TRY(ce_on(&out->ce_initial));
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t step = 0; step < n_steps; ++step) {
        const size_t b = rotate ? ((size_t)step + batch_idx) % nb : batch_idx;  // finetune.zig:171-174
        VKH_TRY(vkh_dataset_batch_seqs(d, b, cfg.n_pos, seqs, in.data(), tg.data()));
        VKH_TRY(vkh_runner_step(r, in.data(), T, tg.data(), T));
    }
    const auto t1 = std::chrono::steady_clock::now();
    out->total_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    out->mean_step_ms = n_steps ? out->total_ms / n_steps : 0.0;
    VKH_TRY(ce_on(&out->ce_final));
    return VKH_OK;
}

}  // extern "C"

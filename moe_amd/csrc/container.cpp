// container.cpp — the two single-file checkpoint containers the reference
// reads, parsed from caller-owned bytes (an mmap'd file):
//   * the packed `.moe` file (src/store.rs:228-279, written by 395-507):
//     "MOEF", u32 version 1, u64 header length, a JSON header whose
//     "tensors" object maps names to {dt, shape, off, len}, then the payload
//     (offsets are relative to the first payload byte, tensors back to back);
//   * GGUF v2/v3 (src/gguf.rs:206-276): metadata key/values, tensor infos
//     (dimensions fastest-first, reversed here), data at the next multiple of
//     general.alignment (default 32).
// Every length read from the file is checked against the buffer before it
// is used, as the reference checks them (a corrupt header is an error, never
// an out-of-bounds read).  Host code only; no GPU involved.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <new>
#include <string>
#include <vector>

#include "../../include/moe_hip.h"

namespace moe {
int fail(int code, const char *fmt, ...);
}

namespace {

using moe::fail;

// The reference's Q6 (6.5 bits per value, no GGUF number): listed with
// this code, which no kernel accepts.
constexpr int32_t kDtQ6 = MOE_DT_Q6_REF;

struct Rec {
    std::string name;
    int32_t dt;
    uint64_t slabs, rows, cols, offset;
};

// a * b, or UINT64_MAX when it does not fit: sizes come from file headers,
// and a corrupt one must not wrap into a small size that then passes a
// bounds check (the reference saturates for the same reason,
// src/store.rs:36-43).
uint64_t sat_mul(uint64_t a, uint64_t b) {
    uint64_t r;
    return __builtin_mul_overflow(a, b, &r) ? UINT64_MAX : r;
}

uint64_t row_bytes_of(int32_t dt, uint64_t cols) {
    switch (dt) {
    case MOE_DT_F32: return sat_mul(cols, 4);
    case MOE_DT_F16:
    case MOE_DT_BF16: return sat_mul(cols, 2);
    case MOE_DT_Q4_0: return cols / 32 * 18;
    case MOE_DT_Q5_0: return cols / 32 * 22;
    case MOE_DT_Q8_0: return cols / 32 * 34;
    case 12: return cols / 256 * 144;  // Q4_K (readable by the reference, not by these kernels)
    case 14: return cols / 256 * 210;  // Q6_K
    case kDtQ6: return cols / 32 * 26;  // the reference's own Q6 (src/quant.rs:81)
    default: return 0;
    }
}

// Saturating slabs * rows * row_bytes (src/store.rs:36-43).
uint64_t rec_len(const Rec &r) { return sat_mul(sat_mul(r.slabs, r.rows), row_bytes_of(r.dt, r.cols)); }

bool fits(const Rec &r, uint64_t len) {
    const uint64_t n = rec_len(r);
    return r.offset <= len && n <= len - r.offset;
}

// ------------------------------------------------------------------ JSON
// Enough JSON for the .moe header: objects, arrays, strings (escapes kept
// as written except \" and \\), numbers, true/false/null.  Values are
// parsed into a small tree; the raw text span of every value is kept so the
// "config" object can be handed back verbatim.
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    bool is_uint = false;
    uint64_t u = 0;
    std::string s;
    std::vector<std::pair<std::string, JVal>> obj;
    std::vector<JVal> arr;
    size_t begin = 0, end = 0;
    const JVal *get(const char *k) const {
        for (auto &kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char *p;
    size_t n, i = 0;
    int depth = 0;
    std::string err;
    void ws() {
        while (i < n && (p[i] == ' ' || p[i] == '\n' || p[i] == '\r' || p[i] == '\t')) i++;
    }
    bool fail_(const char *m) {
        if (err.empty()) err = m;
        return false;
    }
    bool str(std::string &out) {
        if (i >= n || p[i] != '"') return fail_("expected a string");
        i++;
        while (i < n && p[i] != '"') {
            if (p[i] == '\\') {
                if (i + 1 >= n) return fail_("truncated escape");
                const char c = p[i + 1];
                if (c == 'u') {
                    if (i + 6 > n) return fail_("truncated escape");
                    out.append(p + i, 6);  // names in these headers are ASCII; keep the escape as written
                    i += 6;
                    continue;
                }
                out.push_back(c == 'n' ? '\n' : c == 't' ? '\t' : c == 'r' ? '\r' : c == 'b' ? '\b'
                              : c == 'f' ? '\f' : c);
                i += 2;
            } else {
                out.push_back(p[i++]);
            }
        }
        if (i >= n) return fail_("unterminated string");
        i++;
        return true;
    }
    bool val(JVal &v) {
        if (++depth > 256) return fail_("nesting too deep");
        ws();
        if (i >= n) return fail_("unexpected end of header");
        v.begin = i;
        const char c = p[i];
        bool ok = true;
        if (c == '{') {
            v.kind = JVal::Obj;
            i++;
            ws();
            if (i < n && p[i] == '}') {
                i++;
            } else {
                for (;;) {
                    ws();
                    std::string k;
                    if (!str(k)) return false;
                    ws();
                    if (i >= n || p[i] != ':') return fail_("expected ':'");
                    i++;
                    v.obj.emplace_back(std::move(k), JVal{});
                    if (!val(v.obj.back().second)) return false;
                    ws();
                    if (i < n && p[i] == ',') {
                        i++;
                        continue;
                    }
                    if (i < n && p[i] == '}') {
                        i++;
                        break;
                    }
                    return fail_("expected ',' or '}'");
                }
            }
        } else if (c == '[') {
            v.kind = JVal::Arr;
            i++;
            ws();
            if (i < n && p[i] == ']') {
                i++;
            } else {
                for (;;) {
                    v.arr.emplace_back();
                    if (!val(v.arr.back())) return false;
                    ws();
                    if (i < n && p[i] == ',') {
                        i++;
                        continue;
                    }
                    if (i < n && p[i] == ']') {
                        i++;
                        break;
                    }
                    return fail_("expected ',' or ']'");
                }
            }
        } else if (c == '"') {
            v.kind = JVal::Str;
            ok = str(v.s);
        } else if (c == 't' && n - i >= 4 && !memcmp(p + i, "true", 4)) {
            v.kind = JVal::Bool, v.b = true, i += 4;
        } else if (c == 'f' && n - i >= 5 && !memcmp(p + i, "false", 5)) {
            v.kind = JVal::Bool, i += 5;
        } else if (c == 'n' && n - i >= 4 && !memcmp(p + i, "null", 4)) {
            i += 4;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = JVal::Num;
            const size_t s0 = i;
            bool integral = c != '-';
            uint64_t u = 0;
            bool overflow = false;
            while (i < n && (p[i] == '-' || p[i] == '+' || p[i] == '.' || p[i] == 'e' || p[i] == 'E' ||
                             (p[i] >= '0' && p[i] <= '9'))) {
                if (p[i] >= '0' && p[i] <= '9') {
                    if (u > (UINT64_MAX - 9) / 10) overflow = true;
                    u = u * 10 + (uint64_t)(p[i] - '0');
                } else if (i > s0 || p[i] != '-') {
                    integral = false;
                }
                i++;
            }
            v.num = strtod(std::string(p + s0, i - s0).c_str(), nullptr);
            v.is_uint = integral && !overflow;
            v.u = u;
        } else {
            ok = fail_("unexpected character in header");
        }
        v.end = i;
        depth--;
        return ok;
    }
};

int32_t moe_dt_from_name(const std::string &s) {
    std::string u;
    for (char c : s) u.push_back((char)(c >= 'a' && c <= 'z' ? c - 32 : c));
    if (u == "F32") return MOE_DT_F32;
    if (u == "F16") return MOE_DT_F16;
    if (u == "BF16") return MOE_DT_BF16;
    if (u == "Q8") return MOE_DT_Q8_0;
    if (u == "Q4") return MOE_DT_Q4_0;
    if (u == "Q5") return MOE_DT_Q5_0;
    if (u == "Q6") return kDtQ6;
    return MOE_DT_F32;  // what the reference assumes for a name it does not parse
}

// ------------------------------------------------------------------ GGUF
struct Cur {
    const uint8_t *b;
    uint64_t n, at;
    bool take(uint64_t k, const uint8_t *&out) {
        if (k > n || at > n - k) return false;
        out = b + at;
        at += k;
        return true;
    }
    bool u32(uint32_t &v) {
        const uint8_t *q;
        if (!take(4, q)) return false;
        memcpy(&v, q, 4);
        return true;
    }
    bool u64(uint64_t &v) {
        const uint8_t *q;
        if (!take(8, q)) return false;
        memcpy(&v, q, 8);
        return true;
    }
    bool str(std::string &s) {
        uint64_t len;
        const uint8_t *q;
        if (!u64(len) || !take(len, q)) return false;
        s.assign((const char *)q, (size_t)len);
        return true;
    }
};

// Skips (or reads as an integer, for general.alignment) one metadata value
// of GGUF type `t` (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
// 8 string, 9 array, 10 u64, 11 i64, 12 f64).
bool gguf_value(Cur &c, uint32_t t, int depth, int64_t *as_int) {
    static const uint8_t size_of[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (t > 12) return false;
    if (t == 8) {
        std::string s;
        return c.str(s);
    }
    if (t == 9) {
        uint32_t et;
        uint64_t cnt;
        if (depth > 2 || !c.u32(et) || !c.u64(cnt) || cnt > c.n) return false;
        if (et <= 12 && et != 8 && et != 9) {
            const uint8_t *q;
            const unsigned __int128 bytes = (unsigned __int128)cnt * size_of[et];
            return bytes <= c.n && c.take((uint64_t)bytes, q);
        }
        for (uint64_t i = 0; i < cnt; i++)
            if (!gguf_value(c, et, depth + 1, nullptr)) return false;
        return true;
    }
    const uint8_t *q;
    if (!c.take(size_of[t], q)) return false;
    if (as_int) {
        uint64_t v = 0;
        memcpy(&v, q, size_of[t]);
        *as_int = (int64_t)v;
    }
    return true;
}

}  // namespace

struct moe_container {
    int kind = 0;
    std::vector<Rec> recs;
    std::string config;
};

namespace {

int open_moe(const uint8_t *b, uint64_t len, moe_container &c) {
    if (len < 16 || memcmp(b, "MOEF", 4) != 0) return fail(MOE_EINVAL, "not a .moe file");
    uint32_t ver;
    uint64_t hlen;
    memcpy(&ver, b + 4, 4);
    memcpy(&hlen, b + 8, 8);
    if (ver != 1) return fail(MOE_EINVAL, "packed format v%u, this build reads v1", ver);
    if (hlen > len - 16) return fail(MOE_EINVAL, "header claims %llu bytes in a %llu-byte file",
                                     (unsigned long long)hlen, (unsigned long long)len);
    const uint64_t data = 16 + hlen;
    JParser jp{reinterpret_cast<const char *>(b + 16), (size_t)hlen};
    JVal root;
    if (!jp.val(root) || root.kind != JVal::Obj) return fail(MOE_EINVAL, "bad header: %s", jp.err.c_str());
    if (const JVal *cfg = root.get("config"))
        c.config.assign(reinterpret_cast<const char *>(b + 16) + cfg->begin, cfg->end - cfg->begin);
    const JVal *ts = root.get("tensors");
    if (ts && ts->kind == JVal::Obj) {
        for (auto &kv : ts->obj) {
            const JVal &v = kv.second;
            const JVal *dt = v.get("dt"), *shape = v.get("shape"), *off = v.get("off");
            // Dt::parse(..).unwrap_or(Dt::F32), as src/store.rs:245 reads it.
            Rec r{kv.first, (dt && dt->kind == JVal::Str) ? moe_dt_from_name(dt->s) : MOE_DT_F32, 1, 1, 0, 0};
            std::vector<uint64_t> dims;
            if (shape && shape->kind == JVal::Arr)
                for (auto &d : shape->arr)
                    if (d.kind == JVal::Num && d.is_uint) dims.push_back(d.u);
            if (dims.size() == 3)
                r.slabs = dims[0], r.rows = dims[1], r.cols = dims[2];
            else if (dims.size() == 2)
                r.rows = dims[0], r.cols = dims[1];
            else
                continue;  // the reference skips tensors of other ranks
            const uint64_t o = (off && off->kind == JVal::Num && off->is_uint) ? off->u : 0;
            if (o > UINT64_MAX - data) return fail(MOE_EINVAL, "%s: offset overflows", kv.first.c_str());
            r.offset = o + data;
            if (r.dt >= 0 && !fits(r, len))
                return fail(MOE_EINVAL, "%s: %llu bytes at offset %llu runs past the file", kv.first.c_str(),
                            (unsigned long long)rec_len(r), (unsigned long long)r.offset);
            c.recs.push_back(std::move(r));
        }
    }
    c.kind = 1;
    return MOE_OK;
}

int open_gguf(const uint8_t *b, uint64_t len, moe_container &c) {
    Cur cur{b, len, 4};
    uint32_t ver;
    uint64_t n_tensors, n_meta;
    if (!cur.u32(ver)) return fail(MOE_EINVAL, "truncated GGUF header");
    if (ver < 2 || ver > 3) return fail(MOE_EINVAL, "GGUF v%u; this build reads v2 and v3", ver);
    if (!cur.u64(n_tensors) || !cur.u64(n_meta)) return fail(MOE_EINVAL, "truncated GGUF header");
    if (n_tensors > len || n_meta > len) return fail(MOE_EINVAL, "header counts exceed the file size");
    int64_t align = 32;
    for (uint64_t i = 0; i < n_meta; i++) {
        std::string key;
        uint32_t t;
        if (!cur.str(key) || !cur.u32(t)) return fail(MOE_EINVAL, "truncated GGUF metadata");
        int64_t iv = 0;
        const bool is_align = key == "general.alignment" && (t == 4 || t == 5 || t == 10 || t == 11);
        if (!gguf_value(cur, t, 0, is_align ? &iv : nullptr))
            return fail(MOE_EINVAL, "bad or truncated GGUF metadata value for %s", key.c_str());
        if (is_align && iv > 0) align = iv;
    }
    std::vector<Rec> infos;
    for (uint64_t i = 0; i < n_tensors; i++) {
        Rec r{};
        uint32_t dims, t;
        if (!cur.str(r.name) || !cur.u32(dims)) return fail(MOE_EINVAL, "truncated GGUF tensor info");
        if (dims == 0 || dims > 4) return fail(MOE_EINVAL, "%s has %u dimensions", r.name.c_str(), dims);
        uint64_t d[4];
        for (uint32_t j = 0; j < dims; j++)
            if (!cur.u64(d[j])) return fail(MOE_EINVAL, "truncated GGUF tensor info");
        uint64_t off;
        if (!cur.u32(t) || !cur.u64(off)) return fail(MOE_EINVAL, "truncated GGUF tensor info");
        // Fastest-varying dimension first in the file; outermost first here.
        r.cols = d[0];
        r.rows = dims >= 2 ? d[1] : 1;
        r.slabs = dims >= 3 ? d[2] : 1;
        if (dims == 4) r.slabs = sat_mul(r.slabs, d[3]);
        r.dt = (int32_t)t;
        r.offset = off;
        infos.push_back(std::move(r));
    }
    const uint64_t a = (uint64_t)align;
    const uint64_t data = (cur.at + a - 1) / a * a;
    if (data > len) return fail(MOE_EINVAL, "the header runs past the end of the file");
    for (Rec &r : infos) {
        if (r.offset > UINT64_MAX - data) return fail(MOE_EINVAL, "%s: offset overflows", r.name.c_str());
        r.offset += data;
        if (row_bytes_of(r.dt, r.cols) > 0 && !fits(r, len))
            return fail(MOE_EINVAL, "%s: %llu bytes at offset %llu runs past the file", r.name.c_str(),
                        (unsigned long long)rec_len(r), (unsigned long long)r.offset);
    }
    c.recs = std::move(infos);
    c.kind = 2;
    return MOE_OK;
}

void to_public(const Rec &r, moe_rec *o) {
    o->name = r.name.c_str();
    o->dt = r.dt;
    o->_reserved = 0;
    o->slabs = r.slabs;
    o->rows = r.rows;
    o->cols = r.cols;
    o->offset = r.offset;
    o->bytes = row_bytes_of(r.dt, r.cols) > 0 ? rec_len(r) : 0;
}

}  // namespace

extern "C" {

int moe_container_open(const void *bytes, uint64_t len, moe_container **out) {
    if (!out || (!bytes && len)) return fail(MOE_EINVAL, "moe_container_open: bad argument");
    *out = nullptr;
    const uint8_t *b = static_cast<const uint8_t *>(bytes);
    moe_container *c = new (std::nothrow) moe_container;
    if (!c) return fail(MOE_ENOMEM, "moe_container_open: out of memory");
    int rc;
    if (len >= 4 && !memcmp(b, "MOEF", 4))
        rc = open_moe(b, len, *c);
    else if (len >= 4 && !memcmp(b, "GGUF", 4))
        rc = open_gguf(b, len, *c);
    else
        rc = fail(MOE_EINVAL, "neither a .moe nor a GGUF file");
    if (rc) {
        delete c;
        return rc;
    }
    *out = c;
    return MOE_OK;
}

int moe_container_kind(const moe_container *c) { return c ? c->kind : 0; }

int64_t moe_container_count(const moe_container *c) { return c ? (int64_t)c->recs.size() : 0; }

int moe_container_rec(const moe_container *c, int64_t i, moe_rec *out) {
    if (!c || !out || i < 0 || i >= (int64_t)c->recs.size()) return fail(MOE_EINVAL, "moe_container_rec: bad index");
    to_public(c->recs[(size_t)i], out);
    return MOE_OK;
}

int moe_container_find(const moe_container *c, const char *name, moe_rec *out) {
    if (!c || !name || !out) return fail(MOE_EINVAL, "moe_container_find: bad argument");
    for (const Rec &r : c->recs)
        if (r.name == name) {
            to_public(r, out);
            return MOE_OK;
        }
    return fail(MOE_EINVAL, "no tensor named %s", name);
}

const char *moe_container_config(const moe_container *c) {
    return (c && !c->config.empty()) ? c->config.c_str() : nullptr;
}

void moe_container_close(moe_container *c) { delete c; }

int moe_gguf_rename(const char *name, char *out, uint64_t cap) {
    if (!name || !out || cap == 0) return fail(MOE_EINVAL, "moe_gguf_rename: bad argument");
    std::string res;
    const std::string n = name;
    if (n == "token_embd.weight") res = "model.embed_tokens.weight";
    else if (n == "output_norm.weight") res = "model.norm.weight";
    else if (n == "output.weight") res = "lm_head.weight";
    else if (n.compare(0, 4, "blk.") == 0) {
        const size_t dot = n.find('.', 4);
        const std::string layer = dot == std::string::npos ? "" : n.substr(4, dot - 4);
        bool digits = !layer.empty() && layer.size() < 10;
        for (char ch : layer) digits = digits && ch >= '0' && ch <= '9';
        if (digits) {
            const std::string suffix = n.substr(dot + 1);
            static const char *const map[][2] = {
                {"attn_norm.weight", "input_layernorm.weight"},
                {"attn_q_norm.weight", "self_attn.q_norm.weight"},
                {"attn_k_norm.weight", "self_attn.k_norm.weight"},
                {"attn_q.weight", "self_attn.q_proj.weight"},
                {"attn_k.weight", "self_attn.k_proj.weight"},
                {"attn_v.weight", "self_attn.v_proj.weight"},
                {"attn_output.weight", "self_attn.o_proj.weight"},
                {"attn_q.bias", "self_attn.q_proj.bias"},
                {"attn_k.bias", "self_attn.k_proj.bias"},
                {"attn_v.bias", "self_attn.v_proj.bias"},
                {"ffn_norm.weight", "post_attention_layernorm.weight"},
                {"ffn_gate_inp.weight", "mlp.gate.weight"},
                {"exp_probs_b.bias", "mlp.gate.e_score_correction_bias"},
                {"ffn_gate_exps.weight", "mlp.experts.gate_proj"},
                {"ffn_up_exps.weight", "mlp.experts.up_proj"},
                {"ffn_down_exps.weight", "mlp.experts.down_proj"},
                {"ffn_gate_shexp.weight", "mlp.shared_expert.gate_proj.weight"},
                {"ffn_up_shexp.weight", "mlp.shared_expert.up_proj.weight"},
                {"ffn_down_shexp.weight", "mlp.shared_expert.down_proj.weight"},
                {"ffn_gate_inp_shexp.weight", "mlp.shared_expert_gate.weight"},
                {"ffn_gate.weight", "mlp.gate_proj.weight"},
                {"ffn_up.weight", "mlp.up_proj.weight"},
                {"ffn_down.weight", "mlp.down_proj.weight"},
            };
            for (auto &m : map)
                if (suffix == m[0]) {
                    res = "model.layers." + layer + "." + m[1];
                    break;
                }
        }
    }
    if (res.empty()) return 1;  // no counterpart (computed rather than read)
    if (res.size() + 1 > cap) return fail(MOE_EINVAL, "moe_gguf_rename: output buffer too small");
    memcpy(out, res.c_str(), res.size() + 1);
    return MOE_OK;
}

}  // extern "C"

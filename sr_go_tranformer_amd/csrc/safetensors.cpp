// Safetensors archive loader: srq_model_load_safetensors.
//
// Validation restates openHFArchiveFormat (cmd/monolith/monolith.go:648-850,
// cited as M:line) for the Llama / Mistral / Qwen2 profile: the shard index,
// header bounds, duplicate-free JSON (uniqueJSON M:176-228), expected names
// and shapes (hfProfileSpecs M:426-440), dtype widths (hfWidth M:634-642),
// exact extents and gap-free data sections.  Every shard's header is checked
// before the first weight byte is read.  The values then stream from disk
// through a ring of pinned chunks into one device staging buffer and are
// converted / packed on the device by the same kernels as srq_model_load;
// a non-finite value fails with the tensor's name (readTensorValues
// M:884-920).  File reads overlap the device copies and packing: the host
// waits only for the ring slot it is about to refill.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int64_t kMaxHeader = 4 << 20;  // maxHFHeader (M:123)
constexpr int kMaxShards = 128;          // M:741
constexpr int kJsonDepth = 32;           // uniqueJSON (M:185)
constexpr int64_t kJsonNodes = 2000000;
constexpr size_t kChunk = 16 << 20;      // bytes per pinned slot
constexpr int kSlots = 4;

// ------------------------------------------------------------------ JSON
struct JVal {
    enum Type { NUL, BOOL, NUM, STR, ARR, OBJ } t = NUL;
    std::string s;  // STR: decoded text; NUM: the literal
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;
};

// Strict UTF-8 (no overlong forms, no surrogates, at most U+10FFFF).
bool utf8_valid(const unsigned char *p, size_t n) {
    size_t i = 0;
    while (i < n) {
        const unsigned c = p[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        unsigned lo = 0x80, hi = 0xBF;
        if (c >= 0xC2 && c <= 0xDF) len = 2;
        else if (c == 0xE0) len = 3, lo = 0xA0;
        else if (c == 0xED) len = 3, hi = 0x9F;
        else if (c >= 0xE1 && c <= 0xEF) len = 3;
        else if (c == 0xF0) len = 4, lo = 0x90;
        else if (c == 0xF4) len = 4, hi = 0x8F;
        else if (c >= 0xF1 && c <= 0xF3) len = 4;
        else return false;
        if (i + len > n) return false;
        if (p[i + 1] < lo || p[i + 1] > hi) return false;
        for (int k = 2; k < len; ++k)
            if (p[i + k] < 0x80 || p[i + k] > 0xBF) return false;
        i += len;
    }
    return true;
}

void put_utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
        out += (char)cp;
    } else if (cp < 0x800) {
        out += (char)(0xC0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += (char)(0xE0 | (cp >> 12));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    } else {
        out += (char)(0xF0 | (cp >> 18));
        out += (char)(0x80 | ((cp >> 12) & 0x3F));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    }
}

// RFC 8259 parser that rejects duplicate keys (compared after unescaping)
// at every level, nesting deeper than 32, more than 2e6 values and
// anything but whitespace after the document, as uniqueJSON does.
// Unpaired \u surrogates decode to U+FFFD.
class Parser {
  public:
    Parser(const char *p, size_t n) : p_(p), end_(p + n) {}
    bool parse(JVal &root, std::string &err) {
        if (!utf8_valid((const unsigned char *)p_, (size_t)(end_ - p_))) return (err = "invalid JSON UTF-8"), false;
        if (!value(root, 0)) return (err = err_), false;
        ws();
        if (p_ != end_) return (err = "trailing JSON data"), false;
        return true;
    }

  private:
    const char *p_, *end_;
    int64_t nodes_ = 0;
    std::string err_;

    bool bad(const char *what) {
        if (err_.empty()) err_ = what;
        return false;
    }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(end_ - p_) < n || memcmp(p_, w, n) != 0) return bad("invalid JSON literal");
        p_ += n;
        return true;
    }
    static int hexval(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    }
    bool hex4(uint32_t &v) {
        if (end_ - p_ < 4) return bad("invalid JSON escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const int h = hexval(p_[i]);
            if (h < 0) return bad("invalid JSON escape");
            v = v << 4 | (uint32_t)h;
        }
        p_ += 4;
        return true;
    }
    bool str(std::string &out) {
        ++p_;  // opening quote
        out.clear();
        while (true) {
            if (p_ >= end_) return bad("unterminated JSON string");
            const unsigned char c = (unsigned char)*p_;
            if (c == '"') {
                ++p_;
                return true;
            }
            if (c < 0x20) return bad("control character in JSON string");
            if (c != '\\') {
                out += (char)c;
                ++p_;
                continue;
            }
            if (++p_ >= end_) return bad("invalid JSON escape");
            const char e = *p_++;
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t lo = 0;
                        const char *save = p_;
                        if (end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                            p_ += 2;
                            if (!hex4(lo)) return false;
                        }
                        if (lo >= 0xDC00 && lo < 0xE000) {
                            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        } else {
                            cp = 0xFFFD;
                            p_ = save;
                        }
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        cp = 0xFFFD;
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return bad("invalid JSON escape");
            }
        }
    }
    bool num(std::string &out) {
        const char *s = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_) return bad("invalid JSON number");
        if (*p_ == '0') {
            ++p_;
        } else if (*p_ >= '1' && *p_ <= '9') {
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        } else {
            return bad("invalid JSON number");
        }
        if (p_ < end_ && *p_ == '.') {
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return bad("invalid JSON number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return bad("invalid JSON number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        out.assign(s, (size_t)(p_ - s));
        return true;
    }
    bool value(JVal &v, int depth) {
        if (++nodes_ > kJsonNodes || depth > kJsonDepth) return bad("JSON complexity limit");
        ws();
        if (p_ >= end_) return bad("unexpected end of JSON");
        switch (*p_) {
            case '{': {
                v.t = JVal::OBJ;
                ++p_;
                ws();
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                std::unordered_set<std::string> seen;
                while (true) {
                    ws();
                    if (p_ >= end_ || *p_ != '"') return bad("invalid JSON object key");
                    std::string key;
                    if (!str(key)) return false;
                    if (!seen.insert(key).second) return bad("duplicate JSON key");
                    ws();
                    if (p_ >= end_ || *p_ != ':') return bad("invalid JSON object");
                    ++p_;
                    v.o.emplace_back(std::move(key), JVal());
                    if (!value(v.o.back().second, depth + 1)) return false;
                    ws();
                    if (p_ < end_ && *p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (p_ < end_ && *p_ == '}') {
                        ++p_;
                        return true;
                    }
                    return bad("invalid JSON object");
                }
            }
            case '[': {
                v.t = JVal::ARR;
                ++p_;
                ws();
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                while (true) {
                    v.a.emplace_back();
                    if (!value(v.a.back(), depth + 1)) return false;
                    ws();
                    if (p_ < end_ && *p_ == ',') {
                        ++p_;
                        continue;
                    }
                    if (p_ < end_ && *p_ == ']') {
                        ++p_;
                        return true;
                    }
                    return bad("invalid JSON array");
                }
            }
            case '"': v.t = JVal::STR; return str(v.s);
            case 't': v.t = JVal::BOOL, v.s = "true"; return lit("true");
            case 'f': v.t = JVal::BOOL, v.s = "false"; return lit("false");
            case 'n': v.t = JVal::NUL; return lit("null");
            default: v.t = JVal::NUM; return num(v.s);
        }
    }
};


// encoding/json matches struct field names with bytes.EqualFold: ASCII case
// plus the two non-ASCII simple folds of ASCII letters (U+017F long s,
// U+212A Kelvin sign).
std::string fold_key(const std::string &k) {
    std::string out;
    for (size_t i = 0; i < k.size(); ++i) {
        const unsigned char c = (unsigned char)k[i];
        if (c == 0xC5 && i + 1 < k.size() && (unsigned char)k[i + 1] == 0xBF) {
            out += 's', ++i;
        } else if (c == 0xE2 && i + 2 < k.size() && (unsigned char)k[i + 1] == 0x84 &&
                   (unsigned char)k[i + 2] == 0xAA) {
            out += 'k', i += 2;
        } else {
            out += (char)(c >= 'A' && c <= 'Z' ? c + 32 : c);
        }
    }
    return out;
}

// A JSON number as a Go int / int64 (strconv.ParseInt: no fraction, no
// exponent, in range).
bool as_int64(const JVal &v, int64_t &out) {
    if (v.t == JVal::NUL) return (out = 0), true;  // null leaves the zero value
    if (v.t != JVal::NUM) return false;
    const std::string &s = v.s;
    if (s.find_first_of(".eE") != std::string::npos) return false;
    errno = 0;
    char *endp = nullptr;
    const long long x = strtoll(s.c_str(), &endp, 10);
    if (errno == ERANGE || !endp || *endp) return false;
    out = x;
    return true;
}

// Decode a JSON value into a Go []int / []int64 (null: nil slice).
bool as_int_list(const JVal &v, std::vector<int64_t> &out) {
    out.clear();
    if (v.t == JVal::NUL) return true;
    if (v.t != JVal::ARR) return false;
    for (const JVal &e : v.a) {
        int64_t x;
        if (!as_int64(e, x)) return false;
        out.push_back(x);
    }
    return true;
}

// ---------------------------------------------------------------- archive
struct Tensor {
    std::string name;
    int kind = 0, layer = 0;
    std::vector<int64_t> shape;
    int64_t count = 0;
    int shard = -1;           // index into the open files
    int dtype = 0;            // srq_src_dtype
    int64_t width = 0;        // bytes per value
    int64_t off0 = 0, off1 = 0, start = 0;
};

struct Files {
    std::vector<int> fds;
    ~Files() {
        for (int fd : fds) close(fd);
    }
};

// hfProfileSpecs (M:426-440): hfTensorSpecs (M:407-424) in its order, then
// the Qwen2 q/k/v biases per layer, then the untied head.
std::vector<Tensor> profile_specs(const srq_model_config &c) {
    const int64_t d = c.dim, kd = (int64_t)(c.dim / c.heads) * c.kv_heads, h = c.hidden;
    std::vector<Tensor> out;
    auto add = [&](std::string name, int kind, int layer, std::vector<int64_t> shape) {
        Tensor t;
        t.name = std::move(name);
        t.kind = kind, t.layer = layer, t.shape = std::move(shape);
        t.count = 1;
        for (int64_t x : t.shape) t.count *= x;
        out.push_back(std::move(t));
    };
    add("model.embed_tokens.weight", SRQ_T_EMBED, 0, {c.vocab, d});
    for (int i = 0; i < c.layers; ++i) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        add(p + "input_layernorm.weight", SRQ_T_ATTN_NORM, i, {d});
        add(p + "self_attn.q_proj.weight", SRQ_T_Q, i, {d, d});
        add(p + "self_attn.k_proj.weight", SRQ_T_K, i, {kd, d});
        add(p + "self_attn.v_proj.weight", SRQ_T_V, i, {kd, d});
        add(p + "self_attn.o_proj.weight", SRQ_T_O, i, {d, d});
        add(p + "post_attention_layernorm.weight", SRQ_T_FFN_NORM, i, {d});
        add(p + "mlp.gate_proj.weight", SRQ_T_GATE, i, {h, d});
        add(p + "mlp.up_proj.weight", SRQ_T_UP, i, {h, d});
        add(p + "mlp.down_proj.weight", SRQ_T_DOWN, i, {d, h});
    }
    add("model.norm.weight", SRQ_T_FINAL_NORM, 0, {d});
    if (c.qkv_bias) {
        for (int i = 0; i < c.layers; ++i) {
            const std::string p = "model.layers." + std::to_string(i) + ".self_attn.";
            add(p + "q_proj.bias", SRQ_T_Q_BIAS, i, {d});
            add(p + "k_proj.bias", SRQ_T_K_BIAS, i, {kd});
            add(p + "v_proj.bias", SRQ_T_V_BIAS, i, {kd});
        }
    }
    if (!c.tied) add("lm_head.weight", SRQ_T_OUTPUT, 0, {c.vocab, d});
    return out;
}

int read_full(int fd, void *dst, size_t n, int64_t off, const std::string &what) {
    char *p = (char *)dst;
    while (n > 0) {
        const ssize_t r = pread(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r < 0) return fail(SRQ_EFILE, "%s: read failed: %s", what.c_str(), strerror(errno));
        if (r == 0) return fail(SRQ_EFILE, "%s: unexpected end of file", what.c_str());
        p += r, n -= (size_t)r, off += r;
    }
    return SRQ_OK;
}

// readBoundedJSON (M:230-250) for the shard index: a regular file of at most
// maxHFHeader bytes, duplicate-free JSON.
int read_index(const std::string &path, std::vector<std::pair<std::string, std::string>> &weight_map, bool &present) {
    present = false;
    struct stat st;
    if (stat(path.c_str(), &st) != 0) {
        if (errno == ENOENT) return SRQ_OK;
        return fail(SRQ_EFILE, "%s: %s", path.c_str(), strerror(errno));
    }
    present = true;
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(SRQ_EFILE, "%s: %s", path.c_str(), strerror(errno));
    Files guard;
    guard.fds.push_back(fd);
    if (fstat(fd, &st) != 0) return fail(SRQ_EFILE, "%s: %s", path.c_str(), strerror(errno));
    if (!S_ISREG(st.st_mode) || st.st_size > kMaxHeader)
        return fail(SRQ_EFORMAT, "model.safetensors.index.json: metadata size/type limit");
    std::string text((size_t)st.st_size, '\0');
    SRQ_CHECK(read_full(fd, &text[0], text.size(), 0, "model.safetensors.index.json"));
    JVal root;
    std::string err;
    if (!Parser(text.data(), text.size()).parse(root, err))
        return fail(SRQ_EFORMAT, "model.safetensors.index.json: %s", err.c_str());
    // json.Unmarshal into struct{ WeightMap map[string]string }: other keys
    // are ignored; a key folding to "weight_map" decodes into the map (null
    // resets it, an object merges into it).
    if (root.t == JVal::NUL) return SRQ_OK;
    if (root.t != JVal::OBJ) return fail(SRQ_EFORMAT, "model.safetensors.index.json: not a JSON object");
    std::unordered_map<std::string, size_t> at;
    for (const auto &kv : root.o) {
        if (fold_key(kv.first) != "weight_map") continue;
        const JVal &m = kv.second;
        if (m.t == JVal::NUL) {
            weight_map.clear(), at.clear();
            continue;
        }
        if (m.t != JVal::OBJ) return fail(SRQ_EFORMAT, "model.safetensors.index.json: weight_map is not an object");
        for (const auto &e : m.o) {
            if (e.second.t != JVal::STR && e.second.t != JVal::NUL)
                return fail(SRQ_EFORMAT, "model.safetensors.index.json: weight_map value is not a string");
            const std::string file = e.second.t == JVal::STR ? e.second.s : std::string();
            auto it = at.find(e.first);
            if (it != at.end()) {
                weight_map[it->second].second = file;
            } else {
                at[e.first] = weight_map.size();
                weight_map.emplace_back(e.first, file);
            }
        }
    }
    return SRQ_OK;
}

// Decode one header entry into dtype / shape / data_offsets
// (json.Decoder with DisallowUnknownFields, M:790-794).
int decode_entry(const JVal &v, const std::string &name, std::string &dtype, std::vector<int64_t> &shape,
                 std::vector<int64_t> &offsets) {
    dtype.clear(), shape.clear(), offsets.clear();
    if (v.t == JVal::NUL) return SRQ_OK;
    if (v.t != JVal::OBJ) return fail(SRQ_EFORMAT, "HF tensor %s: entry is not a JSON object", name.c_str());
    for (const auto &kv : v.o) {
        const std::string f = fold_key(kv.first);
        if (f == "dtype") {
            if (kv.second.t == JVal::STR) dtype = kv.second.s;
            else if (kv.second.t != JVal::NUL) return fail(SRQ_EFORMAT, "HF tensor %s: dtype is not a string", name.c_str());
        } else if (f == "shape") {
            if (!as_int_list(kv.second, shape))
                return fail(SRQ_EFORMAT, "HF tensor %s: shape is not a list of integers", name.c_str());
        } else if (f == "data_offsets") {
            if (!as_int_list(kv.second, offsets))
                return fail(SRQ_EFORMAT, "HF tensor %s: data_offsets is not a list of integers", name.c_str());
        } else {
            return fail(SRQ_EFORMAT, "HF tensor %s: unknown field \"%s\"", name.c_str(), kv.first.c_str());
        }
    }
    return SRQ_OK;
}

struct DeviceScope {
    int prev = -1;
    explicit DeviceScope(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceScope() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Host and device buffers of one load; released on every exit path after
// the stream has drained.
struct Staging {
    hipStream_t stream = nullptr;
    void *dev = nullptr;
    void *slot[kSlots] = {};
    hipEvent_t done[kSlots] = {};
    bool used[kSlots] = {};
    int32_t *snap = nullptr;  // pinned per-tensor copies of error word 0
    ~Staging() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (dev) (void)hipFree(dev);
        for (int i = 0; i < kSlots; ++i) {
            if (slot[i]) (void)hipHostFree(slot[i]);
            if (done[i]) (void)hipEventDestroy(done[i]);
        }
        if (snap) (void)hipHostFree(snap);
    }
};

// An opened, validated archive: the profile's tensors with their shard,
// dtype and byte range, and the open shard files.
struct Archive {
    std::vector<Tensor> specs;
    std::vector<std::string> shards;
    Files files;
    int64_t total_bytes = 0;
};

// openHFArchiveFormat (M:648-850) for the Llama / Mistral / Qwen2 profile.
int open_archive(const srq_model_config &c, const std::string &root, Archive &a) {
    if (c.vocab < 1 || c.dim < 1 || c.layers < 1 || c.heads < 1 || c.kv_heads < 1 || c.hidden < 1 ||
        c.dim % c.heads != 0)
        return fail(SRQ_EINVAL, "invalid model configuration");
    std::vector<Tensor> &specs = a.specs;
    specs = profile_specs(c);
    std::unordered_map<std::string, int> by_name;
    int64_t parameters = 0;
    for (size_t i = 0; i < specs.size(); ++i) {
        by_name[specs[i].name] = (int)i;
        parameters += specs[i].count;
    }

    // The shard set (M:709-743).
    std::vector<std::pair<std::string, std::string>> weight_map;
    bool indexed = false;
    SRQ_CHECK(read_index(root + "/model.safetensors.index.json", weight_map, indexed));
    std::unordered_map<std::string, std::string> shard_of;
    std::vector<std::string> &shards = a.shards;
    if (indexed) {
        if (weight_map.size() != specs.size()) return fail(SRQ_EFORMAT, "HF shard index tensor count mismatch");
        for (const auto &kv : weight_map) {
            const std::string &file = kv.second;
            const bool plain = !file.empty() && file.find_first_of("/\\") == std::string::npos &&
                               file.size() >= 12 && file.compare(file.size() - 12, 12, ".safetensors") == 0;
            if (!by_name.count(kv.first) || !plain) return fail(SRQ_EFORMAT, "unsupported HF shard index name/path");
            shard_of[kv.first] = file;
            shards.push_back(file);
        }
        std::sort(shards.begin(), shards.end());
        shards.erase(std::unique(shards.begin(), shards.end()), shards.end());
    } else {
        shards.push_back("model.safetensors");
    }
    if (shards.empty() || (int)shards.size() > kMaxShards) return fail(SRQ_EFORMAT, "HF shard count limit");

    // Every shard's header (M:751-849) before any weight byte.
    for (size_t si = 0; si < shards.size(); ++si) {
        const std::string path = root + "/" + shards[si];
        const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) return fail(SRQ_EFILE, "%s: %s", path.c_str(), strerror(errno));
        a.files.fds.push_back(fd);
        struct stat st;
        if (fstat(fd, &st) != 0) return fail(SRQ_EFILE, "%s: %s", path.c_str(), strerror(errno));
        const int64_t size = st.st_size;
        if (!S_ISREG(st.st_mode) || size < 10 || size > parameters * 4 + kMaxHeader + 8)
            return fail(SRQ_EFORMAT, "%s: Safetensors file size/type limit", shards[si].c_str());
        uint8_t prefix[8];
        SRQ_CHECK(read_full(fd, prefix, 8, 0, path));
        uint64_t n = 0;
        for (int b = 7; b >= 0; --b) n = n << 8 | prefix[b];
        if (n < 2 || n > (uint64_t)kMaxHeader || n > (uint64_t)(size - 8))
            return fail(SRQ_EFORMAT, "%s: Safetensors header length limit", shards[si].c_str());
        std::string header((size_t)n, '\0');
        SRQ_CHECK(read_full(fd, &header[0], header.size(), 8, path));
        if (header[0] != '{') return fail(SRQ_EFORMAT, "%s: Safetensors header must start with object", shards[si].c_str());
        JVal hdr;
        std::string err;
        if (!Parser(header.data(), header.size()).parse(hdr, err))
            return fail(SRQ_EFORMAT, "%s: %s", shards[si].c_str(), err.c_str());
        const int64_t data_bytes = size - 8 - (int64_t)n;
        std::vector<Tensor *> ordered;
        for (const auto &kv : hdr.o) {
            if (kv.first == "__metadata__") {
                // json.Unmarshal into map[string]string.
                const JVal &md = kv.second;
                bool ok = md.t == JVal::NUL || md.t == JVal::OBJ;
                if (md.t == JVal::OBJ)
                    for (const auto &e : md.o) ok = ok && (e.second.t == JVal::STR || e.second.t == JVal::NUL);
                if (!ok) return fail(SRQ_EFORMAT, "%s: __metadata__ must map strings to strings", shards[si].c_str());
                continue;
            }
            auto it = by_name.find(kv.first);
            if (it == by_name.end() || specs[it->second].shard >= 0 || (indexed && shard_of[kv.first] != shards[si]))
                return fail(SRQ_EFORMAT, "unexpected or duplicate HF tensor \"%s\"", kv.first.c_str());
            Tensor &t = specs[it->second];
            std::string dtype;
            std::vector<int64_t> shape, offsets;
            SRQ_CHECK(decode_entry(kv.second, t.name, dtype, shape, offsets));
            if (shape != t.shape) return fail(SRQ_EFORMAT, "HF tensor shape mismatch: %s", t.name.c_str());
            const int64_t w = dtype == "F32" ? 4 : (dtype == "F16" || dtype == "BF16") ? 2 : 0;
            if (w == 0 || offsets.size() != 2 || offsets[0] < 0 || offsets[1] < offsets[0] || offsets[1] > data_bytes ||
                offsets[1] - offsets[0] != t.count * w)
                return fail(SRQ_EFORMAT, "invalid HF tensor dtype/extent: %s", t.name.c_str());
            t.shard = (int)si;
            t.width = w;
            t.dtype = dtype == "F32" ? SRQ_SRC_F32 : dtype == "BF16" ? SRQ_SRC_BF16 : SRQ_SRC_F16;
            t.off0 = offsets[0], t.off1 = offsets[1];
            t.start = 8 + (int64_t)n + offsets[0];
            ordered.push_back(&t);
        }
        std::sort(ordered.begin(), ordered.end(), [](const Tensor *a, const Tensor *b) { return a->off0 < b->off0; });
        int64_t end = 0;
        for (const Tensor *t : ordered) {
            if (t->off0 != end) return fail(SRQ_EFORMAT, "%s: Safetensors overlapping or unindexed bytes", shards[si].c_str());
            end = t->off1;
        }
        if (end != data_bytes) return fail(SRQ_EFORMAT, "%s: Safetensors trailing/unindexed bytes", shards[si].c_str());
        a.total_bytes += size;
    }
    for (const Tensor &t : specs)
        if (t.shard < 0) return fail(SRQ_EFORMAT, "missing HF tensor \"%s\"", t.name.c_str());

    return SRQ_OK;
}

}  // namespace
}  // namespace srq

using namespace srq;

extern "C" int srq_archive_check(const srq_model_config *c, const char *dir, int64_t *source_bytes) {
    if (!c || !dir) return fail(SRQ_EINVAL, "null pointer");
    Archive a;
    SRQ_CHECK(open_archive(*c, dir, a));
    if (source_bytes) *source_bytes = a.total_bytes;
    return SRQ_OK;
}

extern "C" int srq_model_load_safetensors(srq_model *m, const char *dir, const volatile int32_t *cancel,
                                          int64_t *source_bytes) {
    if (!m || !dir) return fail(SRQ_EINVAL, "null pointer");
    Archive a;
    SRQ_CHECK(open_archive(model_config(m), dir, a));
    const std::vector<Tensor> &specs = a.specs;
    const std::vector<std::string> &shards = a.shards;
    Files &files = a.files;
    const int64_t total_bytes = a.total_bytes;

    // Stream the values: shard by shard in file order (sequential reads).
    std::vector<const Tensor *> order;
    int64_t largest = 0;
    for (const Tensor &t : specs) {
        order.push_back(&t);
        largest = std::max(largest, t.off1 - t.off0);
    }
    std::sort(order.begin(), order.end(), [](const Tensor *x, const Tensor *y) {
        return x->shard != y->shard ? x->shard < y->shard : x->off0 < y->off0;
    });
    DeviceScope scope(model_device(m));
    Staging sg;
    sg.stream = model_stream(m);
    if (hipMalloc(&sg.dev, (size_t)std::max<int64_t>(largest, 256)) != hipSuccess)
        return fail(SRQ_ENOMEM, "device staging of %lld bytes does not fit", (long long)largest);
    for (int i = 0; i < kSlots; ++i) {
        if (hipHostMalloc(&sg.slot[i], kChunk, hipHostMallocDefault) != hipSuccess)
            return fail(SRQ_ENOMEM, "pinned staging of %zu bytes failed", kChunk);
        SRQ_HIP(hipEventCreateWithFlags(&sg.done[i], hipEventDisableTiming));
    }
    if (hipHostMalloc((void **)&sg.snap, order.size() * sizeof(int32_t), hipHostMallocDefault) != hipSuccess)
        return fail(SRQ_ENOMEM, "pinned flags failed");
    memset(sg.snap, 0, order.size() * sizeof(int32_t));
    const int32_t *err_word = model_error_word(m);
    int chunk = 0;
    size_t issued = 0;
    int rc = SRQ_OK;
    for (; issued < order.size() && rc == SRQ_OK; ++issued) {
        const Tensor &t = *order[issued];
        // Error word 0 is sticky: a set copy of an earlier tensor ends the
        // load early (the join below names the first such tensor).
        if (issued > 0 && ((volatile int32_t *)sg.snap)[issued - 1]) break;
        const int64_t bytes = t.off1 - t.off0;
        for (int64_t pos = 0; pos < bytes && rc == SRQ_OK; pos += (int64_t)kChunk, ++chunk) {
            if (cancel && *cancel) {
                rc = fail(SRQ_ECANCELED, "load canceled");
                break;
            }
            const int s = chunk % kSlots;
            if (sg.used[s] && hipEventSynchronize(sg.done[s]) != hipSuccess) {
                rc = fail(SRQ_EDEVICE, "staging copy failed");
                break;
            }
            const size_t len = (size_t)std::min<int64_t>((int64_t)kChunk, bytes - pos);
            rc = read_full(files.fds[t.shard], sg.slot[s], len, t.start + pos, shards[t.shard]);
            if (rc != SRQ_OK) break;
            if (hipMemcpyAsync((char *)sg.dev + pos, sg.slot[s], len, hipMemcpyHostToDevice, sg.stream) != hipSuccess ||
                hipEventRecord(sg.done[s], sg.stream) != hipSuccess) {
                rc = fail(SRQ_EDEVICE, "staging copy failed");
                break;
            }
            sg.used[s] = true;
        }
        if (rc != SRQ_OK) break;
        rc = model_load_enqueue(m, t.kind, t.layer, sg.dev, t.dtype);
        if (rc == SRQ_OK &&
            hipMemcpyAsync(&sg.snap[issued], err_word, sizeof(int32_t), hipMemcpyDeviceToHost, sg.stream) != hipSuccess)
            rc = fail(SRQ_EDEVICE, "error word copy failed");
    }
    if (hipStreamSynchronize(sg.stream) != hipSuccess && rc == SRQ_OK) rc = fail(SRQ_EDEVICE, "load stream failed");
    // Tensors are consumed in order, so a non-finite tensor fails the load
    // ahead of any later read error or cancellation, as a sequential reader
    // would.
    for (size_t i = 0; i < issued; ++i) {
        if (sg.snap[i]) {
            const std::string what = "non-finite HF weight in " + order[i]->name;
            return model_join_nonfinite(m, what.c_str());
        }
    }
    if (rc != SRQ_OK) {
        const std::string msg = srq_last_error();
        (void)model_join_nonfinite(m, msg.c_str());  // leaves the error word clear
        return fail(rc, "%s", msg.c_str());
    }
    if (source_bytes) *source_bytes = total_bytes;
    return SRQ_OK;
}

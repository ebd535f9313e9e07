// pkv_json.cpp -- host half of the legacy JSON code envelope and of the
// fib-quant digests.
//
// Before the compact TQW1 / FB1 records, proveKV stored a vector's code as
// the serde_json text of turbo-quant's TurboCode or fib-quant's FibCodeV1,
// and the adapters still read that text when a payload lacks the record
// magic (proveKV/src/codec.rs:386-393 turbo decode; 552-561
// FibQuantAdapter::decode_batch_compact; 622-630 decode; 650-658
// decode_batch).  This file restates, for exactly those two structs:
//   - serde_json 1.0.150's reader (from_slice over #[derive(Deserialize)]
//     structs: a JSON object with the fields in any order, unknown fields
//     skipped, a duplicate or missing field an error, or a JSON array of the
//     fields in declaration order; number conversion as its default,
//     non-float_roundtrip parser does it; nothing but whitespace after the
//     value);
//   - the checks the adapters apply after parsing: PolarCode::validate_for
//     (turbo-quant/src/polar.rs:107-152, through PolarQuantizer::decode) and
//     FibQuantizer::validate_code_header (fib-quant/src/codec.rs:926-975)
//     plus the packed-index and norm lengths of decode / decode_batch_fast
//     (codec.rs:506-537, 797-844; bitpack.rs:47-90);
//   - serde_json's writer for the digest views validate_code_header compares
//     against: FibQuantProfileV1::digest (profile.rs:256-262),
//     StoredRotation::digest (rotation.rs:80-100) and
//     FibCodebookV1::compute_digest (codebook.rs:133-157), all through
//     json_digest (digest.rs:5-13): "blake3:" + hex(blake3(domain || 0 ||
//     compact JSON)).
// The hashing uses the same BLAKE3 compression the digest kernels run.
#include <algorithm>
#include <array>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "pkv_blake3.h"
#include "pkv_internal.h"

namespace pkv {
namespace {

// ------------------------------------------------------------------ BLAKE3
// The unkeyed hash with a 32-byte output: chunk chaining values merged on a
// stack as each completed subtree closes, the root flag on the last
// compression (the specification's incremental form).
void blake3_host(const uint8_t* data, size_t len, uint8_t out[32]) {
    using namespace b3;
    const uint64_t nchunks = chunks_of(len);
    std::vector<std::array<uint32_t, 8>> stack;
    for (uint64_t c = 0; c < nchunks; ++c) {
        const size_t off = static_cast<size_t>(c) * CHUNK_BYTES;
        const size_t clen = std::min<size_t>(CHUNK_BYTES, len - off);
        const size_t nblocks = clen == 0 ? 1 : (clen + BLOCK_BYTES - 1) / BLOCK_BYTES;
        const bool last = c + 1 == nchunks;
        uint32_t cv[8];
        set_iv(cv);
        for (size_t b = 0; b < nblocks; ++b) {
            uint8_t buf[64] = {0};
            const size_t blen = std::min<size_t>(BLOCK_BYTES, clen - b * BLOCK_BYTES);
            if (blen) std::memcpy(buf, data + off + b * BLOCK_BYTES, blen);
            uint32_t m[16];
            for (int i = 0; i < 16; ++i)
                m[i] = static_cast<uint32_t>(buf[4 * i]) | (static_cast<uint32_t>(buf[4 * i + 1]) << 8) |
                       (static_cast<uint32_t>(buf[4 * i + 2]) << 16) | (static_cast<uint32_t>(buf[4 * i + 3]) << 24);
            uint32_t flags = (b == 0 ? CHUNK_START : 0u) | (b + 1 == nblocks ? CHUNK_END : 0u);
            if (nchunks == 1 && b + 1 == nblocks) flags |= ROOT;
            compress(cv, m, c, static_cast<uint32_t>(blen), flags);
        }
        std::array<uint32_t, 8> cur;
        std::copy(cv, cv + 8, cur.begin());
        if (last) {
            // fold the stack into the last chunk's value, the bottom merge as root
            for (size_t i = stack.size(); i-- > 0;) {
                uint32_t l[8];
                std::copy(stack[i].begin(), stack[i].end(), l);
                parent(l, cur.data(), i == 0 ? ROOT : 0u);
                std::copy(l, l + 8, cur.begin());
            }
        } else {
            uint64_t total = c + 1;
            while ((total & 1) == 0) {
                uint32_t l[8];
                std::copy(stack.back().begin(), stack.back().end(), l);
                stack.pop_back();
                parent(l, cur.data(), 0u);
                std::copy(l, l + 8, cur.begin());
                total >>= 1;
            }
            stack.push_back(cur);
        }
        if (last) {
            for (int i = 0; i < 8; ++i)
                for (int b = 0; b < 4; ++b) out[4 * i + b] = static_cast<uint8_t>(cur[i] >> (8 * b));
        }
    }
}

std::string digest_text(const std::string& domain, const std::string& json) {
    std::string bytes = domain;
    bytes.push_back('\0');
    bytes += json;
    uint8_t h[32];
    blake3_host(reinterpret_cast<const uint8_t*>(bytes.data()), bytes.size(), h);
    static const char* hex = "0123456789abcdef";
    std::string out = "blake3:";
    for (uint8_t v : h) {
        out.push_back(hex[v >> 4]);
        out.push_back(hex[v & 15]);
    }
    return out;
}

// ------------------------------------------------------------------ writer
// serde_json's text of a float: "null" when not finite; otherwise the
// shortest decimal digits that read back to the same value (the closest such
// string), laid out as the ryu crate's printer lays them out -- which the
// zmij crate behind serde_json 1.0.150's writer keeps: with kk the decimal
// exponent after the last digit's position, plain digits and ".0" up to 16
// (f64) / 13 (f32) integer digits, a decimal point inside the digits, "0."
// and leading zeros down to 1e-5, else d.ddd "e" exponent (no '+', no
// padding).  std::to_chars gives the shortest round-trip digits.
template <typename F>
void put_float(std::string& out, F v) {
    if (!std::isfinite(v)) {
        out += "null";
        return;
    }
    if (v == F(0)) {
        out += std::signbit(v) ? "-0.0" : "0.0";
        return;
    }
    char buf[64];
    const auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
    std::string sci(buf, r.ptr);
    if (sci[0] == '-') {
        out.push_back('-');
        sci.erase(0, 1);
    }
    const size_t e = sci.find('e');
    std::string digits;
    for (size_t i = 0; i < e; ++i)
        if (sci[i] != '.') digits.push_back(sci[i]);
    const int exp10 = std::atoi(sci.c_str() + e + 1);
    const int length = static_cast<int>(digits.size());
    const int kk = exp10 + 1;   // 10^(kk-1) <= |v| < 10^kk
    const int k = kk - length;
    const int lim = sizeof(F) == 8 ? 16 : 13;
    if (k >= 0 && kk <= lim) {
        out += digits;
        out.append(static_cast<size_t>(k), '0');
        out += ".0";
    } else if (kk > 0 && kk <= lim) {
        out += digits.substr(0, static_cast<size_t>(kk));
        out.push_back('.');
        out += digits.substr(static_cast<size_t>(kk));
    } else if (kk > -5 && kk <= 0) {
        out += "0.";
        out.append(static_cast<size_t>(-kk), '0');
        out += digits;
    } else {
        out.push_back(digits[0]);
        if (length > 1) {
            out.push_back('.');
            out += digits.substr(1);
        }
        out.push_back('e');
        out += std::to_string(kk - 1);
    }
}

void put_str(std::string& out, const char* s) {   // ASCII identifiers and constants only
    out.push_back('"');
    out += s;
    out.push_back('"');
}
void put_key(std::string& out, const char* k, bool first = false) {
    if (!first) out.push_back(',');
    put_str(out, k);
    out.push_back(':');
}
void put_u64(std::string& out, uint64_t v) { out += std::to_string(v); }

// FibQuantProfileV1 of FibQuantAdapter::build_quantizer (proveKV/src/codec.rs:
// 471-499): paper_default (profile.rs:132-173) with the adapter's training
// overrides, fields in declaration order (profile.rs:95-130).
std::string fib_profile_json(const pkv_codec_params& p) {
    std::string o = "{";
    const uint32_t wbits = 32u - static_cast<uint32_t>(__builtin_clz(p.n - 1));
    put_key(o, "schema_version", true);
    put_str(o, "fib_quant_profile_v1");
    put_key(o, "ambient_dim");
    put_u64(o, p.dim);
    put_key(o, "block_dim");
    put_u64(o, p.k);
    put_key(o, "codebook_size");
    put_u64(o, p.n);
    put_key(o, "paper_rate_bits_per_coord");
    put_float(o, std::log2(static_cast<double>(p.n)) / static_cast<double>(p.k));
    put_key(o, "wire_index_bits");
    put_u64(o, wbits);
    put_key(o, "wire_bits_per_coord");
    put_float(o, static_cast<double>(wbits) / static_cast<double>(p.k));
    put_key(o, "norm_format");
    put_str(o, "fp16_paper");
    put_key(o, "rotation_seed");
    put_u64(o, p.seed);
    put_key(o, "rotation_algorithm_version");
    put_str(o, "qr-gaussian-chacha8-sign-corrected-v1");
    put_key(o, "codebook_seed");
    put_u64(o, p.seed + 0x9e3779b97f4a7c15ull);
    put_key(o, "codebook_version");
    put_str(o, "fib-quant:paper-core-v1");
    put_key(o, "source_mode");
    put_str(o, "canonical_spherical_beta");
    put_key(o, "radius_method");
    put_str(o, p.k == 2 ? "k2_closed_form" : "beta_quantile");
    put_key(o, "direction_method");
    put_str(o, p.k == 2 ? "fibonacci_spiral" : (p.k == 3 ? "fibonacci_sphere" : "roberts_kronecker"));
    put_key(o, "lloyd_restarts");
    put_u64(o, p.lloyd_restarts);
    put_key(o, "lloyd_iterations");
    put_u64(o, p.lloyd_iterations);
    put_key(o, "training_samples");
    put_u64(o, p.training_samples);
    put_key(o, "empty_cell_policy");
    put_str(o, "split_highest_distortion");
    o.push_back('}');
    return o;
}

// The parameters FibQuantProfileV1::validate accepts (profile.rs:175-254)
// that the digest views here are written for.
bool fib_params_valid(const pkv_codec_params& p) {
    if (p.kind != PKV_CODEC_FIB || p.dim == 0 || p.k == 0 || p.k >= p.dim || p.dim % p.k != 0) return false;
    if (p.n < 2 || p.dim > 16384 || p.k > 256 || p.n > (1u << 20)) return false;
    if (p.lloyd_restarts == 0 || p.lloyd_restarts > 1024) return false;
    if (p.lloyd_iterations == 0 || p.lloyd_iterations > 100000) return false;
    return p.training_samples >= p.n && p.training_samples <= 10000000u;
}

struct FibDigests {
    std::string profile, rotation, codebook;   // codebook: empty until first asked for
};
using DigestKey = std::tuple<uint32_t, uint32_t, uint32_t, uint64_t, uint32_t, uint32_t, uint32_t>;
std::mutex g_dig_mu;
std::map<DigestKey, FibDigests> g_digests;

DigestKey digest_key(const pkv_codec_params& p) {
    return DigestKey(p.dim, p.k, p.n, p.seed, p.training_samples, p.lloyd_restarts, p.lloyd_iterations);
}

// which: 0 profile, 1 rotation, 2 codebook.  Memoised per profile and process
// (the codebook digest runs the host Lloyd build once, for its report).
int fib_digest(const pkv_codec_params& p, int which, std::string* out) {
    if (!fib_params_valid(p)) return PKV_ERR_INVALID_ARG;
    const DigestKey key = digest_key(p);
    {
        std::lock_guard<std::mutex> lock(g_dig_mu);
        auto it = g_digests.find(key);
        if (it != g_digests.end()) {
            const std::string& v = which == 0 ? it->second.profile
                                              : (which == 1 ? it->second.rotation : it->second.codebook);
            if (!v.empty()) {
                *out = v;
                return PKV_OK;
            }
        }
    }
    FibDigests d;
    d.profile = digest_text("fib_quant_profile_v1", fib_profile_json(p));
    std::vector<double> rot;
    int rc = make_fib_rotation(p.dim, p.seed, rot);
    if (rc) return rc;
    {   // StoredRotation::digest's view (rotation.rs:82-98): the row-major matrix
        std::string o = "{";
        put_key(o, "rotation_schema", true);
        put_str(o, "fib_rotation_v1");
        put_key(o, "algorithm_version");
        put_str(o, "qr-gaussian-chacha8-sign-corrected-v1");
        put_key(o, "dim");
        put_u64(o, p.dim);
        put_key(o, "seed");
        put_u64(o, p.seed);
        put_key(o, "matrix");
        o.push_back('[');
        for (size_t i = 0; i < rot.size(); ++i) {
            if (i) o.push_back(',');
            put_float(o, rot[i]);
        }
        o += "]}";
        d.rotation = digest_text("fib_rotation_v1", o);
    }
    if (which == 2) {   // FibCodebookV1::compute_digest's view (codebook.rs:135-156)
        std::vector<float> cb;
        LloydReport rep;
        rc = fib_codebook_report(p.dim, p.k, p.n, p.seed, p.training_samples, p.lloyd_restarts, p.lloyd_iterations,
                                 cb, rep);
        if (rc) return rc;
        std::string o = "{";
        put_key(o, "schema_version", true);
        put_str(o, "fib_codebook_v1");
        put_key(o, "profile_digest");
        put_str(o, d.profile.c_str());
        put_key(o, "rotation_digest");
        put_str(o, d.rotation.c_str());
        put_key(o, "codewords");
        o.push_back('[');
        for (size_t i = 0; i < cb.size(); ++i) {
            if (i) o.push_back(',');
            put_float(o, cb[i]);
        }
        o.push_back(']');
        put_key(o, "init_mse");
        put_float(o, rep.init_mse);
        put_key(o, "training_mse");
        put_float(o, rep.best_mse);
        put_key(o, "refinement_report");   // LloydReportV1 (lloyd.rs:37-59)
        o.push_back('{');
        put_key(o, "schema_version", true);
        put_str(o, "lloyd_report_v1");
        put_key(o, "restarts");
        put_u64(o, rep.restarts);
        put_key(o, "iterations");
        put_u64(o, rep.iterations);
        put_key(o, "training_samples");
        put_u64(o, rep.training_samples);
        put_key(o, "init_mse");
        put_float(o, rep.init_mse);
        put_key(o, "best_mse");
        put_float(o, rep.best_mse);
        put_key(o, "best_restart");
        put_u64(o, rep.best_restart);
        put_key(o, "empty_cells_repaired");
        put_u64(o, rep.repairs);
        put_key(o, "repair_events");
        o.push_back('[');
        for (size_t i = 0; i < rep.events.size(); ++i) {   // LloydRepairEventV1 (lloyd.rs:17-34)
            const LloydRepairEvent& ev = rep.events[i];
            if (i) o.push_back(',');
            o.push_back('{');
            put_key(o, "restart", true);
            put_u64(o, ev.restart);
            put_key(o, "iteration");
            put_u64(o, ev.iteration);
            put_key(o, "empty_cell");
            put_u64(o, ev.empty_cell);
            put_key(o, "donor_cell");
            put_u64(o, ev.donor_cell);
            put_key(o, "donor_count_before");
            put_u64(o, ev.donor_count_before);
            put_key(o, "donor_distortion");
            put_float(o, ev.donor_distortion);
            put_key(o, "residual_norm");
            put_float(o, ev.residual_norm);
            put_key(o, "split_epsilon");
            put_float(o, 1.0e-6);
            o.push_back('}');
        }
        o.push_back(']');
        put_key(o, "seed");
        put_u64(o, rep.seed);
        o += "}}";
        d.codebook = digest_text("fib_codebook_v1", o);
    }
    std::lock_guard<std::mutex> lock(g_dig_mu);
    FibDigests& slot = g_digests[key];
    slot.profile = d.profile;
    slot.rotation = d.rotation;
    if (!d.codebook.empty()) slot.codebook = d.codebook;
    *out = which == 0 ? slot.profile : (which == 1 ? slot.rotation : slot.codebook);
    return PKV_OK;
}

// ------------------------------------------------------------------ reader
// The JSON text as a tree of tokens; strings and numbers keep their source
// span and are converted only where a struct field reads them, as serde_json
// converts only what it deserializes (a skipped field is checked for syntax
// alone).
struct Node {
    enum Type : uint8_t { NUL, TRUE_, FALSE_, NUM, STR, ARR, OBJ } t = NUL;
    size_t a = 0, b = 0;             // NUM: the token; STR: the bytes between the quotes
    std::vector<uint32_t> kids;      // ARR: elements; OBJ: key, value, key, value, ...
};

struct Doc {
    const uint8_t* s = nullptr;
    size_t n = 0;
    std::vector<Node> nodes;
};

bool is_ws(uint8_t c) { return c == ' ' || c == '\n' || c == '\t' || c == '\r'; }
bool is_digit(uint8_t c) { return c >= '0' && c <= '9'; }
bool is_hex(uint8_t c) { return is_digit(c) || (c >= 'a' && c <= 'f') || (c >= 'A' && c <= 'F'); }

// A string token starting at the opening quote: escapes must be one of
// \" \\ \/ \b \f \n \r \t \uXXXX and no byte below 0x20 may appear (serde_json
// rejects both, also in skipped strings).  i ends after the closing quote.
bool scan_string(const Doc& d, size_t& i, size_t* a, size_t* b) {
    ++i;
    *a = i;
    while (i < d.n) {
        const uint8_t c = d.s[i];
        if (c == '"') {
            *b = i;
            ++i;
            return true;
        }
        if (c < 0x20) return false;
        if (c == '\\') {
            if (++i >= d.n) return false;
            const uint8_t e = d.s[i];
            if (e == 'u') {
                if (i + 4 >= d.n) return false;
                for (int k = 1; k <= 4; ++k)
                    if (!is_hex(d.s[i + k])) return false;
                i += 4;
            } else if (!std::strchr("\"\\/bfnrt", e) || e == 0) {
                return false;
            }
        }
        ++i;
    }
    return false;
}

// JSON number grammar: -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?
bool scan_number(const Doc& d, size_t& i) {
    if (i < d.n && d.s[i] == '-') ++i;
    if (i >= d.n || !is_digit(d.s[i])) return false;
    if (d.s[i] == '0') {
        ++i;
        if (i < d.n && is_digit(d.s[i])) return false;   // one leading zero only
    } else {
        while (i < d.n && is_digit(d.s[i])) ++i;
    }
    if (i < d.n && d.s[i] == '.') {
        ++i;
        if (i >= d.n || !is_digit(d.s[i])) return false;
        while (i < d.n && is_digit(d.s[i])) ++i;
    }
    if (i < d.n && (d.s[i] == 'e' || d.s[i] == 'E')) {
        ++i;
        if (i < d.n && (d.s[i] == '+' || d.s[i] == '-')) ++i;
        if (i >= d.n || !is_digit(d.s[i])) return false;
        while (i < d.n && is_digit(d.s[i])) ++i;
    }
    return true;
}

// serde_json::from_slice's syntax pass: one value, then only whitespace.
// Iterative, so nesting depth inside skipped fields is not limited by the
// host stack (serde_json skips them iteratively too).
bool parse_doc(Doc& d, uint32_t* root) {
    size_t i = 0;
    std::vector<uint32_t> open;
    bool want_value = true;
    auto ws = [&] { while (i < d.n && is_ws(d.s[i])) ++i; };
    auto attach = [&](uint32_t idx) {
        if (!open.empty()) d.nodes[open.back()].kids.push_back(idx);
    };
    auto key = [&]() -> bool {   // an object key (a string) and its ':'
        ws();
        if (i >= d.n || d.s[i] != '"') return false;
        Node k;
        k.t = Node::STR;
        if (!scan_string(d, i, &k.a, &k.b)) return false;
        d.nodes.push_back(k);
        attach(static_cast<uint32_t>(d.nodes.size() - 1));
        ws();
        if (i >= d.n || d.s[i] != ':') return false;
        ++i;
        return true;
    };
    for (;;) {
        if (want_value) {
            ws();
            if (i >= d.n) return false;
            const uint8_t c = d.s[i];
            const uint32_t idx = static_cast<uint32_t>(d.nodes.size());
            d.nodes.emplace_back();
            attach(idx);
            if (c == '{' || c == '[') {
                d.nodes[idx].t = c == '{' ? Node::OBJ : Node::ARR;
                ++i;
                open.push_back(idx);
                ws();
                if (i < d.n && d.s[i] == (c == '{' ? '}' : ']')) {
                    ++i;
                    open.pop_back();
                    want_value = false;
                    continue;
                }
                if (c == '{' && !key()) return false;
                continue;
            }
            Node& v = d.nodes[idx];
            if (c == '"') {
                v.t = Node::STR;
                if (!scan_string(d, i, &v.a, &v.b)) return false;
            } else if (c == '-' || is_digit(c)) {
                v.t = Node::NUM;
                v.a = i;
                if (!scan_number(d, i)) return false;
                v.b = i;
            } else if (d.n - i >= 4 && std::memcmp(d.s + i, "null", 4) == 0) {
                v.t = Node::NUL;
                i += 4;
            } else if (d.n - i >= 4 && std::memcmp(d.s + i, "true", 4) == 0) {
                v.t = Node::TRUE_;
                i += 4;
            } else if (d.n - i >= 5 && std::memcmp(d.s + i, "false", 5) == 0) {
                v.t = Node::FALSE_;
                i += 5;
            } else {
                return false;
            }
            want_value = false;
            continue;
        }
        ws();
        if (open.empty()) {
            if (i != d.n) return false;   // trailing characters
            *root = 0;
            return !d.nodes.empty();
        }
        if (i >= d.n) return false;
        const Node& top = d.nodes[open.back()];
        const uint8_t close = top.t == Node::OBJ ? '}' : ']';
        if (d.s[i] == ',') {
            ++i;
            if (top.t == Node::OBJ && !key()) return false;
            want_value = true;
        } else if (d.s[i] == close) {
            ++i;
            open.pop_back();
        } else {
            return false;
        }
    }
}

// A string value as serde_json's parse_str returns it: escapes decoded, a
// \u surrogate pair joined (a lone surrogate is an error), and the result
// valid UTF-8.
bool utf8_ok(const std::string& s) {
    size_t i = 0;
    while (i < s.size()) {
        const uint8_t c = static_cast<uint8_t>(s[i]);
        int len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (!len || i + len > s.size()) return false;
        uint32_t cp = len == 1 ? c : c & (0x7f >> len);
        for (int k = 1; k < len; ++k) {
            const uint8_t cc = static_cast<uint8_t>(s[i + k]);
            if ((cc >> 6) != 2) return false;
            cp = (cp << 6) | (cc & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)) ||
            (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += len;
    }
    return true;
}
void put_utf8(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
        o.push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
        o.push_back(static_cast<char>(0xC0 | (cp >> 6)));
        o.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
        o.push_back(static_cast<char>(0xE0 | (cp >> 12)));
        o.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
        o.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
        o.push_back(static_cast<char>(0xF0 | (cp >> 18)));
        o.push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
        o.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
        o.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
}
uint32_t hex4(const uint8_t* p) {
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
        const uint8_t c = p[k];
        v = v * 16 + (is_digit(c) ? c - '0' : (c | 0x20) - 'a' + 10);
    }
    return v;
}
bool string_value(const Doc& d, const Node& v, std::string* out) {
    if (v.t != Node::STR) return false;
    std::string o;
    for (size_t i = v.a; i < v.b; ++i) {
        const uint8_t c = d.s[i];
        if (c != '\\') {
            o.push_back(static_cast<char>(c));
            continue;
        }
        const uint8_t e = d.s[++i];
        switch (e) {
        case '"': o.push_back('"'); break;
        case '\\': o.push_back('\\'); break;
        case '/': o.push_back('/'); break;
        case 'b': o.push_back('\b'); break;
        case 'f': o.push_back('\f'); break;
        case 'n': o.push_back('\n'); break;
        case 'r': o.push_back('\r'); break;
        case 't': o.push_back('\t'); break;
        default: {   // 'u'
            uint32_t cp = hex4(d.s + i + 1);
            i += 4;
            if (cp >= 0xDC00 && cp <= 0xDFFF) return false;   // lone trailing surrogate
            if (cp >= 0xD800 && cp <= 0xDBFF) {
                if (i + 6 >= v.b || d.s[i + 1] != '\\' || d.s[i + 2] != 'u') return false;
                const uint32_t lo = hex4(d.s + i + 3);
                if (lo < 0xDC00 || lo > 0xDFFF) return false;
                cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                i += 6;
            }
            put_utf8(o, cp);
        }
        }
    }
    if (!utf8_ok(o)) return false;
    *out = std::move(o);
    return true;
}

// serde_json's ParserNumber of a number token (its default parser: the
// significand accumulated in a u64, further digits dropped into the
// exponent, the value significand * or / 10^|exp| in f64 with 10^308 steps
// below that; an overflowing positive exponent is an error, not infinity).
struct Number {
    enum Kind { U64, I64, F64 } kind = U64;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
};
const double* pow10_table() {
    static const std::vector<double> t = [] {
        std::vector<double> v(309);
        char buf[16];
        for (int e = 0; e <= 308; ++e) {
            std::snprintf(buf, sizeof buf, "1e%d", e);
            v[e] = std::strtod(buf, nullptr);   // correctly rounded
        }
        return v;
    }();
    return t.data();
}
bool f64_from_parts(bool positive, uint64_t significand, int32_t exponent, double* out) {
    const double* pow10 = pow10_table();
    double f = static_cast<double>(significand);
    for (;;) {
        const uint32_t mag = exponent == INT32_MIN ? 0x80000000u : static_cast<uint32_t>(exponent < 0 ? -exponent : exponent);
        if (mag <= 308) {
            if (exponent >= 0) {
                f *= pow10[mag];
                if (std::isinf(f)) return false;
            } else {
                f /= pow10[mag];
            }
            break;
        }
        if (f == 0.0) break;
        if (exponent >= 0) return false;
        f /= 1e308;
        exponent += 308;
    }
    *out = positive ? f : -f;
    return true;
}
bool overflows10(uint64_t a, uint64_t digit, uint64_t max) { return a >= max / 10 && (a > max / 10 || digit > max % 10); }
bool number_value(const Doc& d, const Node& v, Number* out) {
    if (v.t != Node::NUM) return false;
    size_t i = v.a;
    const size_t end = v.b;
    const bool positive = d.s[i] != '-';
    if (!positive) ++i;
    uint64_t sig = 0;
    int32_t exponent = 0;
    bool is_float = false, dropped = false;
    // integer part
    for (; i < end && is_digit(d.s[i]); ++i) {
        const uint64_t dg = d.s[i] - '0';
        if (dropped || overflows10(sig, dg, UINT64_MAX)) {   // parse_long_integer
            dropped = true;
            is_float = true;
            ++exponent;
        } else {
            sig = sig * 10 + dg;
        }
    }
    if (i < end && d.s[i] == '.') {   // parse_decimal
        is_float = true;
        ++i;
        for (; i < end && is_digit(d.s[i]); ++i) {
            const uint64_t dg = d.s[i] - '0';
            if (dropped || overflows10(sig, dg, UINT64_MAX)) {   // parse_decimal_overflow
                dropped = true;
                continue;
            }
            sig = sig * 10 + dg;
            --exponent;
        }
    }
    if (i < end && (d.s[i] == 'e' || d.s[i] == 'E')) {   // parse_exponent
        is_float = true;
        ++i;
        bool pos_exp = true;
        if (d.s[i] == '+') ++i;
        else if (d.s[i] == '-') { pos_exp = false; ++i; }
        int32_t e = 0;
        for (; i < end; ++i) {
            const uint64_t dg = d.s[i] - '0';
            if (overflows10(static_cast<uint64_t>(e), dg, INT32_MAX)) {   // parse_exponent_overflow
                if (sig != 0 && pos_exp) return false;
                out->kind = Number::F64;
                out->f = positive ? 0.0 : -0.0;
                return true;
            }
            e = e * 10 + static_cast<int32_t>(dg);
        }
        const int64_t fe = static_cast<int64_t>(exponent) + (pos_exp ? e : -static_cast<int64_t>(e));
        exponent = static_cast<int32_t>(std::max<int64_t>(INT32_MIN, std::min<int64_t>(INT32_MAX, fe)));
    }
    if (is_float) {
        out->kind = Number::F64;
        return f64_from_parts(positive, sig, exponent, &out->f);
    }
    if (positive) {
        out->kind = Number::U64;
        out->u = sig;
        return true;
    }
    const int64_t neg = static_cast<int64_t>(0 - sig);   // (significand as i64).wrapping_neg()
    if (neg >= 0) {   // -0, or below i64::MIN: a float
        out->kind = Number::F64;
        out->f = -static_cast<double>(sig);
    } else {
        out->kind = Number::I64;
        out->i = neg;
    }
    return true;
}

// serde's primitive visitors over a ParserNumber.
bool de_unsigned(const Doc& d, const Node& v, uint64_t max, uint64_t* out) {
    Number x;
    if (!number_value(d, v, &x) || x.kind != Number::U64 || x.u > max) return false;
    *out = x.u;
    return true;
}
bool de_signed(const Doc& d, const Node& v, int64_t lo, int64_t hi, int64_t* out) {
    Number x;
    if (!number_value(d, v, &x)) return false;
    if (x.kind == Number::U64) {
        if (x.u > static_cast<uint64_t>(hi)) return false;
        *out = static_cast<int64_t>(x.u);
        return true;
    }
    if (x.kind == Number::I64 && x.i >= lo && x.i <= hi) {
        *out = x.i;
        return true;
    }
    return false;
}
bool de_f32(const Doc& d, const Node& v, float* out) {
    Number x;
    if (!number_value(d, v, &x)) return false;
    *out = x.kind == Number::U64 ? static_cast<float>(x.u)
                                 : (x.kind == Number::I64 ? static_cast<float>(x.i) : static_cast<float>(x.f));
    return true;
}
bool de_seq(const Node& v, std::vector<uint32_t>* items) {
    if (v.t != Node::ARR) return false;
    *items = v.kids;
    return true;
}

// A #[derive(Deserialize)] struct: from an object (keys decoded and matched
// by name, unknown ones skipped, a repeated known field or a missing one an
// error) or from an array holding exactly the fields in declaration order.
bool de_struct(const Doc& d, const Node& v, const char* const* names, int nf, uint32_t* fields) {
    if (v.t == Node::ARR) {
        if (static_cast<int>(v.kids.size()) != nf) return false;
        for (int f = 0; f < nf; ++f) fields[f] = v.kids[f];
        return true;
    }
    if (v.t != Node::OBJ) return false;
    std::vector<bool> seen(nf, false);
    for (size_t k = 0; k + 1 < v.kids.size(); k += 2) {
        std::string name;
        if (!string_value(d, d.nodes[v.kids[k]], &name)) return false;
        for (int f = 0; f < nf; ++f) {
            if (name == names[f]) {
                if (seen[f]) return false;   // duplicate field
                seen[f] = true;
                fields[f] = v.kids[k + 1];
            }
        }
    }
    for (int f = 0; f < nf; ++f)
        if (!seen[f]) return false;   // missing field
    return true;
}

// ------------------------------------------------------------------ codes
void put_bits(uint8_t* dst, uint64_t bitpos, uint32_t bits, uint32_t value) {   // LSB-first
    for (uint32_t b = 0; b < bits; ++b, ++bitpos)
        if ((value >> b) & 1u) dst[bitpos >> 3] |= static_cast<uint8_t>(1u << (bitpos & 7));
}

// TurboCode {polar_code: PolarCode, residual_sketch: QjlSketch}
// (turbo-quant/src/turbo.rs:50-56, polar.rs:35-46, qjl.rs:41-50), checked as
// PolarQuantizer::new(dim, bits - 1, seed).decode does (validate_for), then
// written as the payload of the equivalent TQW1 record: f32 radii, packed
// angle indices, and the sketch's signs when it holds one per projection
// (the decode never reads them).
int turbo_from_json(const pkv_codec_params& p, const Doc& d, uint32_t root, std::vector<uint8_t>* payload,
                    int* stage) {
    static const char* const top[] = {"polar_code", "residual_sketch"};
    static const char* const pc[] = {"dim", "bits", "radii", "angle_indices"};
    static const char* const qs[] = {"dim", "projections", "signs"};
    uint32_t tf[2], pf[4], qf[3];
    *stage = 1;
    if (!de_struct(d, d.nodes[root], top, 2, tf)) return PKV_ERR_CORRUPT_PAYLOAD;
    if (!de_struct(d, d.nodes[tf[0]], pc, 4, pf)) return PKV_ERR_CORRUPT_PAYLOAD;
    uint64_t cdim, cbits;
    if (!de_unsigned(d, d.nodes[pf[0]], UINT64_MAX, &cdim) || !de_unsigned(d, d.nodes[pf[1]], 255, &cbits))
        return PKV_ERR_CORRUPT_PAYLOAD;
    std::vector<uint32_t> items;
    if (!de_seq(d.nodes[pf[2]], &items)) return PKV_ERR_CORRUPT_PAYLOAD;
    std::vector<float> radii(items.size());
    for (size_t t = 0; t < items.size(); ++t)
        if (!de_f32(d, d.nodes[items[t]], &radii[t])) return PKV_ERR_CORRUPT_PAYLOAD;
    if (!de_seq(d.nodes[pf[3]], &items)) return PKV_ERR_CORRUPT_PAYLOAD;
    std::vector<uint32_t> angles(items.size());
    for (size_t t = 0; t < items.size(); ++t) {
        uint64_t a;
        if (!de_unsigned(d, d.nodes[items[t]], 65535, &a)) return PKV_ERR_CORRUPT_PAYLOAD;
        angles[t] = static_cast<uint32_t>(a);
    }
    if (!de_struct(d, d.nodes[tf[1]], qs, 3, qf)) return PKV_ERR_CORRUPT_PAYLOAD;
    uint64_t sdim, sproj;
    if (!de_unsigned(d, d.nodes[qf[0]], UINT64_MAX, &sdim) || !de_unsigned(d, d.nodes[qf[1]], UINT64_MAX, &sproj))
        return PKV_ERR_CORRUPT_PAYLOAD;
    if (!de_seq(d.nodes[qf[2]], &items)) return PKV_ERR_CORRUPT_PAYLOAD;
    std::vector<int64_t> signs(items.size());
    for (size_t t = 0; t < items.size(); ++t)
        if (!de_signed(d, d.nodes[items[t]], -128, 127, &signs[t])) return PKV_ERR_CORRUPT_PAYLOAD;
    // PolarCode::validate_for(dim, bits - 1) (polar.rs:107-152)
    *stage = 2;
    const uint32_t pbits = p.bits - 1, pairs = p.dim / 2, levels = 1u << pbits;
    if (cdim != p.dim || cbits != pbits) return PKV_ERR_CORRUPT_PAYLOAD;
    if (radii.size() != pairs) return PKV_ERR_CORRUPT_PAYLOAD;
    for (float r : radii)
        if (!std::isfinite(r) || r < 0.0f) return PKV_ERR_CORRUPT_PAYLOAD;
    if (angles.size() != pairs) return PKV_ERR_CORRUPT_PAYLOAD;
    for (uint32_t a : angles)
        if (a >= levels) return PKV_ERR_CORRUPT_PAYLOAD;
    *stage = 0;
    const size_t abytes = (static_cast<size_t>(pairs) * pbits + 7) / 8, sbytes = (p.projections + 7) / 8;
    payload->assign(4 * static_cast<size_t>(pairs) + abytes + sbytes, 0);
    uint8_t* o = payload->data();
    for (uint32_t t = 0; t < pairs; ++t) std::memcpy(o + 4 * t, &radii[t], 4);
    for (uint32_t t = 0; t < pairs; ++t) put_bits(o + 4 * pairs, static_cast<uint64_t>(t) * pbits, pbits, angles[t]);
    if (signs.size() == p.projections)
        for (uint32_t j = 0; j < p.projections; ++j)
            if (signs[j] > 0) put_bits(o + 4 * pairs + abytes, j, 1, 1);
    return PKV_OK;
}

// FibCodeV1 (fib-quant/src/codec.rs:31-54), checked as validate_code_header
// (926-975) and the index / norm lengths decode and decode_batch_fast read
// (bitpack.rs:47-66, codec.rs:1020-1031), then written as the payload of the
// equivalent FB1 record: fp16 norm bytes, packed indices.  Padding bits,
// index range and the norm's value are the record decode's own checks.
int fib_from_json(const pkv_codec_params& p, const Doc& d, uint32_t root, std::vector<uint8_t>* payload, int* stage) {
    static const char* const names[] = {"schema_version", "profile_digest", "codebook_digest", "rotation_digest",
                                        "ambient_dim",    "block_dim",      "norm_format",     "norm_payload",
                                        "wire_index_bits", "block_count",   "indices"};
    uint32_t f[11];
    *stage = 1;
    if (!de_struct(d, d.nodes[root], names, 11, f)) return PKV_ERR_CORRUPT_PAYLOAD;
    std::string schema, pdig, cdig, rdig, nf;
    if (!string_value(d, d.nodes[f[0]], &schema) || !string_value(d, d.nodes[f[1]], &pdig) ||
        !string_value(d, d.nodes[f[2]], &cdig) || !string_value(d, d.nodes[f[3]], &rdig))
        return PKV_ERR_CORRUPT_PAYLOAD;
    uint64_t amb, blk, wbits, count;
    if (!de_unsigned(d, d.nodes[f[4]], UINT32_MAX, &amb) || !de_unsigned(d, d.nodes[f[5]], UINT32_MAX, &blk))
        return PKV_ERR_CORRUPT_PAYLOAD;
    // NormFormat (profile.rs:26-35, snake_case unit variants): "name" or {"name": null}
    const Node& nv = d.nodes[f[6]];
    if (nv.t == Node::STR) {
        if (!string_value(d, nv, &nf)) return PKV_ERR_CORRUPT_PAYLOAD;
    } else if (nv.t == Node::OBJ && nv.kids.size() == 2 && d.nodes[nv.kids[1]].t == Node::NUL) {
        if (!string_value(d, d.nodes[nv.kids[0]], &nf)) return PKV_ERR_CORRUPT_PAYLOAD;
    } else {
        return PKV_ERR_CORRUPT_PAYLOAD;
    }
    if (nf != "fp16_paper" && nf != "f32_reference") return PKV_ERR_CORRUPT_PAYLOAD;
    std::vector<uint32_t> items;
    if (!de_seq(d.nodes[f[7]], &items)) return PKV_ERR_CORRUPT_PAYLOAD;
    std::vector<uint8_t> norm(items.size());
    for (size_t t = 0; t < items.size(); ++t) {
        uint64_t b;
        if (!de_unsigned(d, d.nodes[items[t]], 255, &b)) return PKV_ERR_CORRUPT_PAYLOAD;
        norm[t] = static_cast<uint8_t>(b);
    }
    if (!de_unsigned(d, d.nodes[f[8]], 255, &wbits) || !de_unsigned(d, d.nodes[f[9]], UINT32_MAX, &count))
        return PKV_ERR_CORRUPT_PAYLOAD;
    if (!de_seq(d.nodes[f[10]], &items)) return PKV_ERR_CORRUPT_PAYLOAD;
    std::vector<uint8_t> idx(items.size());
    for (size_t t = 0; t < items.size(); ++t) {
        uint64_t b;
        if (!de_unsigned(d, d.nodes[items[t]], 255, &b)) return PKV_ERR_CORRUPT_PAYLOAD;
        idx[t] = static_cast<uint8_t>(b);
    }
    // validate_code_header (codec.rs:926-975), in its order
    *stage = 2;
    if (schema != "fib_code_v1") return PKV_ERR_CORRUPT_PAYLOAD;
    std::string want;
    int rc = fib_digest(p, 0, &want);
    if (rc) return rc;
    if (pdig != want) return PKV_ERR_CORRUPT_PAYLOAD;                  // ProfileDigestMismatch
    if (!cdig.empty()) {
        if ((rc = fib_digest(p, 2, &want))) return rc;
        if (cdig != want) return PKV_ERR_CORRUPT_PAYLOAD;              // CodebookDigestMismatch
    }
    if (!rdig.empty()) {
        if ((rc = fib_digest(p, 1, &want))) return rc;
        if (rdig != want) return PKV_ERR_CORRUPT_PAYLOAD;              // RotationDigestMismatch
    }
    const uint32_t pwbits = 32u - static_cast<uint32_t>(__builtin_clz(p.n - 1));
    if (amb != p.dim || blk != p.k || count != p.dim / p.k || wbits != pwbits || nf != "fp16_paper")
        return PKV_ERR_CORRUPT_PAYLOAD;
    const size_t ibytes = (static_cast<size_t>(p.dim / p.k) * pwbits + 7) / 8;
    if (idx.size() != ibytes) return PKV_ERR_CORRUPT_PAYLOAD;          // unpack_indices length
    if (norm.size() != 2) return PKV_ERR_CORRUPT_PAYLOAD;              // decode_norm: fp16 length
    *stage = 0;
    payload->assign(norm.begin(), norm.end());
    payload->insert(payload->end(), idx.begin(), idx.end());
    return PKV_OK;
}

}  // namespace

int code_from_json(const pkv_codec_params& p, const uint8_t* json, uint64_t len, std::vector<uint8_t>* payload,
                   int* stage) {
    *stage = 0;
    if (p.kind == PKV_CODEC_TURBO) {
        if (p.dim == 0 || p.dim % 2 || p.bits < 2 || p.bits > 17) return PKV_ERR_INVALID_ARG;
    } else if (!fib_params_valid(p)) {
        return PKV_ERR_INVALID_ARG;
    }
    Doc d;
    d.s = json;
    d.n = static_cast<size_t>(len);
    uint32_t root = 0;
    if (!json || !parse_doc(d, &root)) {
        *stage = 1;
        return PKV_ERR_CORRUPT_PAYLOAD;
    }
    return p.kind == PKV_CODEC_TURBO ? turbo_from_json(p, d, root, payload, stage)
                                     : fib_from_json(p, d, root, payload, stage);
}

}  // namespace pkv

extern "C" {

int pkv_code_from_json(const pkv_codec_params* params, const uint8_t* json, uint64_t len, uint8_t* payload,
                       uint64_t cap, uint64_t* payload_len, int* stage) {
    int st = 0;
    if (stage) *stage = 0;
    if (payload_len) *payload_len = 0;
    if (!params || (!json && len)) return PKV_ERR_INVALID_ARG;
    std::vector<uint8_t> out;
    const int rc = pkv::code_from_json(*params, json, len, &out, &st);
    if (stage) *stage = st;
    if (rc) return rc;
    if (payload_len) *payload_len = out.size();
    if (!payload || cap < out.size()) return PKV_ERR_CAPACITY;
    std::memcpy(payload, out.data(), out.size());
    return PKV_OK;
}

int pkv_fib_digests(const pkv_codec_params* params, char* profile_digest, char* codebook_digest,
                    char* rotation_digest) {
    if (!params) return PKV_ERR_INVALID_ARG;
    char* outs[3] = {profile_digest, rotation_digest, codebook_digest};
    for (int which = 0; which < 3; ++which) {
        if (!outs[which]) continue;
        std::string s;
        const int rc = pkv::fib_digest(*params, which, &s);
        if (rc) return rc;
        std::memcpy(outs[which], s.c_str(), s.size() + 1);
    }
    return PKV_OK;
}

void pkv_host_blake3(const void* data, uint64_t len, uint8_t out[32]) {
    pkv::blake3_host(static_cast<const uint8_t*>(data), static_cast<size_t>(len), out);
}

}  // extern "C"

// checkpoint.hip -- the unchanged MLX safetensors checkpoint on the HIP side
// (src/safetensors.rs:85-196 Checkpoint::open / meta / read_with;
// src/lfm.rs:261-316 load_tensor / load_quant).  Host code: the shard
// headers are parsed once at open (a model.safetensors.index.json names the
// shards, else model.safetensors); a tensor read streams the file through two
// pinned staging buffers into device memory, the next chunk read from disk
// while the previous one is copied.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "mh_host.hpp"

struct mh_checkpoint {
    struct Meta {
        int dtype;  // MH_DTYPE_*, or MH_DTYPE_OTHER
        std::vector<uint64_t> shape;
        uint64_t start, end;  // absolute byte range in the shard
        int shard;
    };
    std::vector<std::string> shards;
    std::map<std::string, Meta> tensors;  // sorted by name
    std::vector<const std::string*> order;
    void* staging[2] = {nullptr, nullptr};
    bool pinned[2] = {false, false};
    hipEvent_t copied[2] = {nullptr, nullptr};
};

namespace {

constexpr size_t kStageBytes = 16u << 20;

int hip_ok(hipError_t e, const char* what) { return e == hipSuccess ? MH_OK : mh::hip_error(e, what); }

// ------------------------------------------------ a small JSON reader ---
// Enough of RFC 8259 for safetensors headers and index files: objects,
// arrays, strings (escapes, \u to UTF-8), integers, other numbers, true /
// false / null.  Values are kept as a tree.
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool is_int = false;
    uint64_t u = 0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const char* key) const {
        for (const auto& kv : obj) {
            if (kv.first == key) {
                return &kv.second;
            }
        }
        return nullptr;
    }
};

struct Parser {
    const char* p;
    const char* e;
    int depth = 0;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) {
            ++p;
        }
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if (static_cast<size_t>(e - p) < n || memcmp(p, w, n) != 0) {
            return false;
        }
        p += n;
        return true;
    }
    static void put_utf8(std::string& out, uint32_t c) {
        if (c < 0x80) {
            out += static_cast<char>(c);
        } else if (c < 0x800) {
            out += static_cast<char>(0xc0 | (c >> 6));
            out += static_cast<char>(0x80 | (c & 0x3f));
        } else if (c < 0x10000) {
            out += static_cast<char>(0xe0 | (c >> 12));
            out += static_cast<char>(0x80 | ((c >> 6) & 0x3f));
            out += static_cast<char>(0x80 | (c & 0x3f));
        } else {
            out += static_cast<char>(0xf0 | (c >> 18));
            out += static_cast<char>(0x80 | ((c >> 12) & 0x3f));
            out += static_cast<char>(0x80 | ((c >> 6) & 0x3f));
            out += static_cast<char>(0x80 | (c & 0x3f));
        }
    }
    bool hex4(uint32_t& v) {
        if (e - p < 4) {
            return false;
        }
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return false;
        }
        return true;
    }
    bool str(std::string& out) {
        if (p >= e || *p != '"') {
            return false;
        }
        ++p;
        while (p < e && *p != '"') {
            const char c = *p++;
            if (static_cast<unsigned char>(c) < 0x20) {
                return false;
            }
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p >= e) {
                return false;
            }
            const char x = *p++;
            switch (x) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t c1;
                    if (!hex4(c1)) return false;
                    if (c1 >= 0xd800 && c1 < 0xdc00) {  // surrogate pair
                        uint32_t c2;
                        if (!lit("\\u") || !hex4(c2) || c2 < 0xdc00 || c2 >= 0xe000) return false;
                        c1 = 0x10000 + ((c1 - 0xd800) << 10) + (c2 - 0xdc00);
                    }
                    put_utf8(out, c1);
                    break;
                }
                default: return false;
            }
        }
        if (p >= e) {
            return false;
        }
        ++p;
        return true;
    }
    bool num(Json& v) {
        const char* b = p;
        if (p < e && *p == '-') ++p;
        bool digits = false, frac = false;
        uint64_t u = 0;
        bool overflow = false;
        while (p < e && *p >= '0' && *p <= '9') {
            const uint64_t d = static_cast<uint64_t>(*p - '0');
            overflow = overflow || u > (UINT64_MAX - d) / 10u;
            u = u * 10u + d;
            ++p;
            digits = true;
        }
        if (p < e && *p == '.') {
            frac = true;
            ++p;
            while (p < e && *p >= '0' && *p <= '9') ++p;
        }
        if (p < e && (*p == 'e' || *p == 'E')) {
            frac = true;
            ++p;
            if (p < e && (*p == '+' || *p == '-')) ++p;
            while (p < e && *p >= '0' && *p <= '9') ++p;
        }
        if (!digits) {
            return false;
        }
        v.kind = Json::NUM;
        v.is_int = !frac && *b != '-' && !overflow;
        v.u = u;
        return true;
    }
    bool value(Json& v) {
        if (++depth > 64) {
            return false;
        }
        ws();
        bool ok = false;
        if (p >= e) {
            ok = false;
        } else if (*p == '{') {
            ++p;
            v.kind = Json::OBJ;
            ws();
            if (p < e && *p == '}') {
                ++p;
                ok = true;
            } else {
                while (true) {
                    ws();
                    std::pair<std::string, Json> kv;
                    if (!str(kv.first)) break;
                    ws();
                    if (p >= e || *p != ':') break;
                    ++p;
                    if (!value(kv.second)) break;
                    v.obj.push_back(std::move(kv));
                    ws();
                    if (p < e && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < e && *p == '}') {
                        ++p;
                        ok = true;
                    }
                    break;
                }
            }
        } else if (*p == '[') {
            ++p;
            v.kind = Json::ARR;
            ws();
            if (p < e && *p == ']') {
                ++p;
                ok = true;
            } else {
                while (true) {
                    Json x;
                    if (!value(x)) break;
                    v.arr.push_back(std::move(x));
                    ws();
                    if (p < e && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < e && *p == ']') {
                        ++p;
                        ok = true;
                    }
                    break;
                }
            }
        } else if (*p == '"') {
            v.kind = Json::STR;
            ok = str(v.s);
        } else if (lit("true") || lit("false")) {
            v.kind = Json::BOOL;
            ok = true;
        } else if (lit("null")) {
            v.kind = Json::NUL;
            ok = true;
        } else {
            ok = num(v);
        }
        --depth;
        return ok;
    }
};

bool parse_json(const std::string& text, Json& out) {
    Parser ps{text.data(), text.data() + text.size()};
    if (!ps.value(out)) {
        return false;
    }
    ps.ws();
    return ps.p == ps.e;
}

bool read_file(const std::string& path, std::string& out) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) {
        return false;
    }
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) {
        out.append(buf, n);
    }
    const bool ok = !ferror(f);
    fclose(f);
    return ok;
}

bool exists(const std::string& path) {
    struct stat st;
    return stat(path.c_str(), &st) == 0;
}

int dtype_of(const std::string& s) {
    if (s == "BF16") return MH_DTYPE_BF16;
    if (s == "F32") return MH_DTYPE_F32;
    if (s == "U32") return MH_DTYPE_U32;
    return MH_DTYPE_OTHER;
}

size_t dtype_size(int d) { return d == MH_DTYPE_BF16 ? 2u : (d == MH_DTYPE_F32 || d == MH_DTYPE_U32) ? 4u : 0u; }

// One shard's header (src/safetensors.rs:160-196): u64 LE length, a JSON
// object of name -> {dtype, shape, data_offsets}; "__metadata__" skipped.
int parse_shard(mh_checkpoint* ck, int shard) {
    const std::string& path = ck->shards[shard];
    FILE* f = fopen(path.c_str(), "rb");
    MH_ENSURE(f != nullptr, MH_ERR_INVALID, "checkpoint: cannot open %s (%s)", path.c_str(), strerror(errno));
    uint8_t lb[8];
    const bool got = fread(lb, 1, 8, f) == 8;
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | lb[i];
    fseek(f, 0, SEEK_END);
    const long fsize = ftell(f);
    std::string header;
    bool ok = got && hlen <= static_cast<uint64_t>(fsize) - 8u && hlen <= (100u << 20);
    if (ok) {
        header.resize(hlen);
        fseek(f, 8, SEEK_SET);
        ok = fread(&header[0], 1, hlen, f) == hlen;
    }
    fclose(f);
    MH_ENSURE(ok, MH_ERR_INVALID, "checkpoint: %s: bad or truncated header", path.c_str());
    Json root;
    MH_ENSURE(parse_json(header, root) && root.kind == Json::OBJ, MH_ERR_INVALID,
              "checkpoint: %s: header is not a JSON object", path.c_str());
    const uint64_t data = 8u + hlen;
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") {
            continue;
        }
        const Json& ent = kv.second;
        const Json* dt = ent.get("dtype");
        const Json* sh = ent.get("shape");
        const Json* off = ent.get("data_offsets");
        MH_ENSURE(ent.kind == Json::OBJ && dt && dt->kind == Json::STR && sh && sh->kind == Json::ARR && off &&
                      off->kind == Json::ARR && off->arr.size() == 2 && off->arr[0].is_int && off->arr[1].is_int,
                  MH_ERR_INVALID, "checkpoint: %s: bad header entry for %s", path.c_str(), kv.first.c_str());
        mh_checkpoint::Meta m;
        m.dtype = dtype_of(dt->s);
        for (const Json& d : sh->arr) {
            MH_ENSURE(d.is_int, MH_ERR_INVALID, "checkpoint: %s: bad shape for %s", path.c_str(), kv.first.c_str());
            m.shape.push_back(d.u);
        }
        MH_ENSURE(m.shape.size() <= MH_MAX_DIMS, MH_ERR_UNSUPPORTED, "checkpoint: %s has %zu dimensions",
                  kv.first.c_str(), m.shape.size());
        const uint64_t a = off->arr[0].u, b = off->arr[1].u;
        MH_ENSURE(b >= a, MH_ERR_INVALID, "checkpoint: tensor %s has reversed data offsets", kv.first.c_str());
        // data <= fsize holds (hlen <= fsize - 8), so the subtraction cannot wrap
        MH_ENSURE(b <= static_cast<uint64_t>(fsize) - data, MH_ERR_INVALID,
                  "checkpoint: tensor %s extends past the end of %s", kv.first.c_str(), path.c_str());
        // the byte range must be exactly the shape's elements (known dtypes):
        // reads copy end - start bytes into buffers sized from the shape
        if (dtype_size(m.dtype) != 0) {
            uint64_t elems = 1;
            bool fits = true;
            for (uint64_t d : m.shape) {
                fits = fits && (d == 0 || elems <= UINT64_MAX / d);
                elems = fits ? elems * d : 0;
            }
            fits = fits && elems <= UINT64_MAX / dtype_size(m.dtype);
            MH_ENSURE(fits && b - a == elems * dtype_size(m.dtype), MH_ERR_INVALID,
                      "checkpoint: tensor %s holds %llu bytes, its shape needs a different count", kv.first.c_str(),
                      static_cast<unsigned long long>(b - a));
        }
        m.start = data + a;
        m.end = data + b;
        m.shard = shard;
        MH_ENSURE(ck->tensors.emplace(kv.first, m).second, MH_ERR_INVALID,
                  "checkpoint: tensor %s appears in multiple shards", kv.first.c_str());
    }
    return MH_OK;
}

const mh_checkpoint::Meta* find(const mh_checkpoint* ck, const char* name) {
    const auto it = ck->tensors.find(name);
    return it == ck->tensors.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

int mh_checkpoint_open(const char* dir, mh_checkpoint** out) {
    MH_ENSURE(dir && out, MH_ERR_INVALID, "mh_checkpoint_open: NULL argument");
    *out = nullptr;
    auto* ck = new mh_checkpoint();
    const std::string d(dir);
    const std::string index = d + "/model.safetensors.index.json";
    int rc = MH_OK;
    if (exists(index)) {
        std::string text;
        Json root;
        if (!read_file(index, text) || !parse_json(text, root) || root.kind != Json::OBJ) {
            rc = mh::set_error(MH_ERR_INVALID, "checkpoint: cannot parse %s", index.c_str());
        } else {
            std::vector<std::string> names;
            const Json* wm = root.get("weight_map");
            if (wm && wm->kind == Json::OBJ) {
                for (const auto& kv : wm->obj) {
                    if (kv.second.kind == Json::STR) names.push_back(kv.second.s);
                }
            }
            std::sort(names.begin(), names.end());
            names.erase(std::unique(names.begin(), names.end()), names.end());
            for (const auto& n : names) ck->shards.push_back(d + "/" + n);
        }
    } else if (exists(d + "/model.safetensors")) {
        ck->shards.push_back(d + "/model.safetensors");
    } else {
        rc = mh::set_error(MH_ERR_INVALID, "checkpoint: no model.safetensors.index.json or model.safetensors under %s",
                           dir);
    }
    for (size_t i = 0; rc == MH_OK && i < ck->shards.size(); ++i) {
        rc = parse_shard(ck, static_cast<int>(i));
    }
    if (rc != MH_OK) {
        delete ck;
        return rc;
    }
    for (const auto& kv : ck->tensors) ck->order.push_back(&kv.first);
    *out = ck;
    return MH_OK;
}

void mh_checkpoint_close(mh_checkpoint* ck) {
    if (!ck) {
        return;
    }
    for (int i = 0; i < 2; ++i) {
        if (ck->copied[i]) (void)hipEventDestroy(ck->copied[i]);
        if (ck->staging[i]) {
            if (ck->pinned[i]) {
                (void)hipHostFree(ck->staging[i]);
            } else {
                free(ck->staging[i]);
            }
        }
    }
    delete ck;
}

uint32_t mh_checkpoint_count(const mh_checkpoint* ck) { return ck ? static_cast<uint32_t>(ck->order.size()) : 0u; }

const char* mh_checkpoint_name(const mh_checkpoint* ck, uint32_t i) {
    return ck && i < ck->order.size() ? ck->order[i]->c_str() : nullptr;
}

int mh_checkpoint_meta(const mh_checkpoint* ck, const char* name, mh_tensor_meta* meta) {
    MH_ENSURE(ck && name && meta, MH_ERR_INVALID, "mh_checkpoint_meta: NULL argument");
    const mh_checkpoint::Meta* m = find(ck, name);
    MH_ENSURE(m != nullptr, MH_ERR_INVALID, "checkpoint: tensor %s not in checkpoint", name);
    memset(meta, 0, sizeof(*meta));
    meta->dtype = m->dtype;
    meta->ndim = static_cast<uint32_t>(m->shape.size());
    for (size_t i = 0; i < m->shape.size(); ++i) meta->shape[i] = m->shape[i];
    meta->bytes = m->end - m->start;
    return MH_OK;
}

int mh_checkpoint_read(mh_checkpoint* ck, const char* name, void* dst, size_t bytes, mh_stream_t stream) {
    MH_ENSURE(ck && name && dst, MH_ERR_INVALID, "mh_checkpoint_read: NULL argument");
    const mh_checkpoint::Meta* m = find(ck, name);
    MH_ENSURE(m != nullptr, MH_ERR_INVALID, "checkpoint: tensor %s not in checkpoint", name);
    MH_ENSURE(dtype_size(m->dtype) != 0, MH_ERR_UNSUPPORTED, "checkpoint: tensor %s has an unsupported dtype", name);
    MH_ENSURE(bytes == m->end - m->start, MH_ERR_INVALID, "checkpoint: destination for %s is %zu bytes, tensor is %llu",
              name, bytes, static_cast<unsigned long long>(m->end - m->start));
    for (int i = 0; i < 2; ++i) {
        if (!ck->staging[i]) {
            // pinned when the runtime grants it (DMA straight from the buffer);
            // otherwise pageable memory, which the runtime copies through its own
            // pinned bounce buffers
            if (hipHostMalloc(&ck->staging[i], kStageBytes, hipHostMallocDefault) == hipSuccess) {
                ck->pinned[i] = true;
            } else {
                (void)hipGetLastError();
                ck->staging[i] = malloc(kStageBytes);
                MH_ENSURE(ck->staging[i] != nullptr, MH_ERR_RUNTIME, "checkpoint: no staging memory");
            }
            MH_TRY(hip_ok(hipEventCreateWithFlags(&ck->copied[i], hipEventDisableTiming), "hipEventCreate"));
        }
    }
    const int fd = open(ck->shards[m->shard].c_str(), O_RDONLY);
    MH_ENSURE(fd >= 0, MH_ERR_INVALID, "checkpoint: cannot open %s (%s)", ck->shards[m->shard].c_str(),
              strerror(errno));
    const hipStream_t s = mh::as_stream(stream);
    int rc = MH_OK;
    size_t done = 0;
    for (int i = 0; rc == MH_OK && done < bytes; i ^= 1) {
        const size_t len = std::min(kStageBytes, bytes - done);
        // the copy that last used this buffer is finished before it is refilled
        rc = hip_ok(hipEventSynchronize(ck->copied[i]), "hipEventSynchronize");
        size_t got = 0;
        while (rc == MH_OK && got < len) {
            const ssize_t r = pread(fd, static_cast<char*>(ck->staging[i]) + got, len - got,
                                    static_cast<off_t>(m->start + done + got));
            if (r <= 0) {
                rc = mh::set_error(MH_ERR_INVALID, "checkpoint: reading %s failed", name);
            } else {
                got += static_cast<size_t>(r);
            }
        }
        if (rc == MH_OK) {
            rc = hip_ok(hipMemcpyAsync(static_cast<char*>(dst) + done, ck->staging[i], len,
                                              hipMemcpyHostToDevice, s),
                               "hipMemcpyAsync");
        }
        if (rc == MH_OK) {
            rc = hip_ok(hipEventRecord(ck->copied[i], s), "hipEventRecord");
        }
        done += len;
    }
    close(fd);
    // the staging buffers stay owned by the checkpoint: the copies are done
    // when this returns
    if (rc == MH_OK) {
        rc = hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
    return rc;
}

int mh_load_quant(mh_checkpoint* ck, const char* base, uint32_t rows, uint32_t k, uint32_t bits, uint32_t* codes,
                  uint16_t* scales, uint16_t* biases, mh_quant_weights* out, mh_stream_t stream) {
    MH_ENSURE(ck && base && codes && scales && biases && out, MH_ERR_INVALID, "mh_load_quant: NULL argument");
    const std::string b(base);
    const mh_checkpoint::Meta* sm = find(ck, (b + ".scales").c_str());
    const mh_checkpoint::Meta* bm = find(ck, (b + ".biases").c_str());
    const mh_checkpoint::Meta* wm = find(ck, (b + ".weight").c_str());
    MH_ENSURE(sm, MH_ERR_INVALID, "missing %s.scales", base);
    MH_ENSURE(bm, MH_ERR_INVALID, "missing %s.biases", base);
    MH_ENSURE(wm, MH_ERR_INVALID, "missing %s.weight", base);
    MH_ENSURE(wm->dtype == MH_DTYPE_U32, MH_ERR_INVALID, "%s codes must be U32", base);
    MH_ENSURE(!wm->shape.empty(), MH_ERR_INVALID, "%s: empty shape", base);
    MH_ENSURE(bits == 4u || bits == 6u || bits == 8u, MH_ERR_UNSUPPORTED, "%s: unsupported bit width %u", base, bits);
    MH_ENSURE(k > 0u && rows > 0u, MH_ERR_INVALID, "%s: empty matrix (%u x %u)", base, rows, k);
    const uint64_t cols = wm->shape.back();
    MH_ENSURE(cols > 0u, MH_ERR_INVALID, "%s: codes have no columns", base);
    MH_ENSURE(k % 64u == 0 && !sm->shape.empty() && sm->shape.back() == k / 64u, MH_ERR_INVALID,
              "%s: scales group count mismatch", base);
    const uint64_t found = 32u * cols / k;
    MH_ENSURE(found == bits, MH_ERR_INVALID, "%s: expected %u-bit, found %llu", base, bits,
              static_cast<unsigned long long>(found));
    uint64_t n = 1, ns = 1, nb = 1;
    for (uint64_t d : wm->shape) n *= d;
    for (uint64_t d : sm->shape) ns *= d;
    for (uint64_t d : bm->shape) nb *= d;
    MH_ENSURE(n / cols == rows, MH_ERR_INVALID, "%s: rows %llu != %u", base, static_cast<unsigned long long>(n / cols),
              rows);
    MH_ENSURE(ns / (k / 64u) == rows && nb / (k / 64u) == rows, MH_ERR_INVALID, "%s: scale rows mismatch", base);
    MH_ENSURE(sm->dtype == MH_DTYPE_BF16 && bm->dtype == MH_DTYPE_BF16, MH_ERR_INVALID, "%s: scales dtype", base);
    // the caller's buffers hold exactly rows x k codes and rows x k/64 scale /
    // bias pairs: every byte range read must be that size
    const uint64_t code_bytes = static_cast<uint64_t>(rows) * k * bits / 8u;
    const uint64_t sb_bytes = static_cast<uint64_t>(rows) * (k / 64u) * 2u;
    MH_ENSURE(wm->end - wm->start == code_bytes && sm->end - sm->start == sb_bytes &&
                  bm->end - bm->start == sb_bytes,
              MH_ERR_INVALID, "%s: tensor byte counts do not match %u x %u at %u bits", base, rows, k, bits);
    MH_TRY(mh_checkpoint_read(ck, (b + ".weight").c_str(), codes, wm->end - wm->start, stream));
    MH_TRY(mh_checkpoint_read(ck, (b + ".scales").c_str(), scales, sm->end - sm->start, stream));
    MH_TRY(mh_checkpoint_read(ck, (b + ".biases").c_str(), biases, bm->end - bm->start, stream));
    out->codes = codes;
    out->scales = scales;
    out->biases = biases;
    out->out_features = rows;
    out->in_features = k;
    out->group_size = 64;
    out->bits = bits;
    return MH_OK;
}

}  // extern "C"

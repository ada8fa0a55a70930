// ckpt.cpp -- checkpoint readers (safetensors, GGUF, titan-v1 INT4 blobs) and
// the load-time repack into the gfx950 TILED layout.  Host code only.
//
// The reference copies stored bytes to the GPU as they are
// (loader.cpp:434-472, gguf_loader.cpp:299-342, moe.cpp:613-724); here a
// quantized weight is read once, repacked on the host with
// titan_repack_host (whose inverse, titan_unpack_host, returns the stored
// bytes exactly) and handed to the caller for a single upload.
#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <functional>
#include <cstdlib>
#include <memory>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "titan_ckpt.h"
#include "titan_qmm.h"

namespace {

// ---- a small JSON reader (safetensors headers, index and manifest files) ----
struct JV {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0;
    bool is_int = false;
    long long i = 0;
    std::string s;
    std::vector<JV> a;
    std::vector<std::pair<std::string, JV>> o;
    const JV* get(const char* key) const {
        if (kind != OBJ) return nullptr;
        for (auto& kv : o)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    bool ok = true;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* w) {
        size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n)) return false;
        p += n;
        return true;
    }
    static void utf8(std::string& out, unsigned cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 63));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 63));
            out += (char)(0x80 | (cp & 63));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 63));
            out += (char)(0x80 | ((cp >> 6) & 63));
            out += (char)(0x80 | (cp & 63));
        }
    }
    bool hex4(unsigned& v) {
        if (end - p < 4) return false;
        v = 0;
        for (int k = 0; k < 4; k++) {
            char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool str(std::string& out) {
        if (p >= end || *p != '"') return false;
        p++;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p >= end) return false;
            char e = *p++;
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
                    unsigned cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        unsigned lo;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: return false;
            }
        }
        if (p >= end) return false;
        p++;
        return true;
    }
    bool value(JV& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p >= end) return false;
        char c = *p;
        if (c == '{') {
            v.kind = JV::OBJ;
            p++;
            ws();
            if (p < end && *p == '}') { p++; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (p >= end || *p != ':') return false;
                p++;
                v.o.emplace_back(std::move(k), JV());
                if (!value(v.o.back().second, depth + 1)) return false;
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == '}') { p++; return true; }
                return false;
            }
        }
        if (c == '[') {
            v.kind = JV::ARR;
            p++;
            ws();
            if (p < end && *p == ']') { p++; return true; }
            for (;;) {
                v.a.emplace_back();
                if (!value(v.a.back(), depth + 1)) return false;
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == ']') { p++; return true; }
                return false;
            }
        }
        if (c == '"') { v.kind = JV::STR; return str(v.s); }
        if (lit("true")) { v.kind = JV::BOOL; v.b = true; return true; }
        if (lit("false")) { v.kind = JV::BOOL; return true; }
        if (lit("null")) return true;
        // number
        const char* q = p;
        if (q < end && (*q == '-' || *q == '+')) q++;
        bool integral = true;
        while (q < end && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' || *q == '-' || *q == '+')) {
            if (*q == '.' || *q == 'e' || *q == 'E') integral = false;
            q++;
        }
        if (q == p) return false;
        std::string t(p, q);
        char* e = nullptr;
        v.kind = JV::NUM;
        v.num = strtod(t.c_str(), &e);
        if (!e || *e) return false;
        if (integral) {
            errno = 0;
            v.i = strtoll(t.c_str(), &e, 10);
            v.is_int = errno == 0 && e && !*e;
        }
        p = q;
        return true;
    }
};

bool parse_json(const std::string& text, JV& out) {
    JsonParser jp{text.data(), text.data() + text.size()};
    if (!jp.value(out, 0)) return false;
    jp.ws();
    return jp.p == jp.end;
}

bool as_u64(const JV* v, uint64_t& out) {
    if (!v || v->kind != JV::NUM || !v->is_int || v->i < 0) return false;
    out = (uint64_t)v->i;
    return true;
}

// ---- files --------------------------------------------------------------------
struct File {
    int fd = -1;
    uint64_t size = 0;
    ~File() {
        if (fd >= 0) close(fd);
    }
};

bool read_at(const File& f, uint64_t off, void* dst, uint64_t n) {
    if (off > f.size || n > f.size - off) return false;
    char* d = (char*)dst;
    uint64_t done = 0;
    while (done < n) {
        ssize_t r = pread(f.fd, d + done, (size_t)std::min<uint64_t>(n - done, 1u << 30), (off_t)(off + done));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        done += (uint64_t)r;
    }
    return true;
}

bool is_dir(const std::string& p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}
bool is_file(const std::string& p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

// Bytes per element of the safetensors / GGUF plain types (0 = unknown).
int ck_elem_bytes(int dt) {
    switch (dt) {
        case TITAN_CK_F64: case TITAN_CK_I64: return 8;
        case TITAN_CK_F32: case TITAN_CK_I32: return 4;
        case TITAN_CK_F16: case TITAN_CK_BF16: case TITAN_CK_I16: return 2;
        case TITAN_CK_I8: case TITAN_CK_U8: case TITAN_CK_BOOL: case TITAN_CK_F8_E4M3: case TITAN_CK_F8_E5M2: return 1;
        default: return 0;
    }
}

int st_dtype(const std::string& s) {
    static const std::pair<const char*, int> tab[] = {
        {"F64", TITAN_CK_F64}, {"F32", TITAN_CK_F32}, {"F16", TITAN_CK_F16}, {"BF16", TITAN_CK_BF16},
        {"I64", TITAN_CK_I64}, {"I32", TITAN_CK_I32}, {"I16", TITAN_CK_I16}, {"I8", TITAN_CK_I8},
        {"U8", TITAN_CK_U8}, {"BOOL", TITAN_CK_BOOL}, {"F8_E4M3", TITAN_CK_F8_E4M3},
        {"F8_E5M2", TITAN_CK_F8_E5M2}};
    for (auto& t : tab)
        if (s == t.first) return t.second;
    return -1;
}

// GGUF / ggml type geometry (gguf_loader.h:29-100, with the public ggml block
// sizes for the types that table leaves at 0): {elements, bytes} per block.
bool ggml_geometry(uint32_t t, int& blk, int& bytes) {
    switch (t) {
        case 0: blk = 1; bytes = 4; return true;      // F32
        case 1: blk = 1; bytes = 2; return true;      // F16
        case 2: blk = 32; bytes = 18; return true;    // Q4_0
        case 3: blk = 32; bytes = 20; return true;    // Q4_1
        case 6: blk = 32; bytes = 22; return true;    // Q5_0
        case 7: blk = 32; bytes = 24; return true;    // Q5_1
        case 8: blk = 32; bytes = 34; return true;    // Q8_0
        case 9: blk = 32; bytes = 36; return true;    // Q8_1
        case 10: blk = 256; bytes = 84; return true;  // Q2_K
        case 11: blk = 256; bytes = 110; return true; // Q3_K
        case 12: blk = 256; bytes = 144; return true; // Q4_K
        case 13: blk = 256; bytes = 176; return true; // Q5_K
        case 14: blk = 256; bytes = 210; return true; // Q6_K
        case 15: blk = 256; bytes = 292; return true; // Q8_K
        case 24: blk = 1; bytes = 1; return true;     // I8
        case 25: blk = 1; bytes = 2; return true;     // I16
        case 26: blk = 1; bytes = 4; return true;     // I32
        case 27: blk = 1; bytes = 8; return true;     // I64
        case 28: blk = 1; bytes = 8; return true;     // F64
        case 30: blk = 1; bytes = 2; return true;     // BF16
        default: return false;
    }
}
int ggml_plain_dtype(uint32_t t) {
    switch (t) {
        case 0: return TITAN_CK_F32;
        case 1: return TITAN_CK_F16;
        case 24: return TITAN_CK_I8;
        case 25: return TITAN_CK_I16;
        case 26: return TITAN_CK_I32;
        case 27: return TITAN_CK_I64;
        case 28: return TITAN_CK_F64;
        case 30: return TITAN_CK_BF16;
        default: return TITAN_CK_GGML;
    }
}

struct Tensor {
    std::string name;
    int dtype = -1, ggml_type = -1, ndim = 0, group_size = 0;
    int64_t shape[8] = {0};
    int file = 0;
    uint64_t offset = 0, nbytes = 0;
};

}  // namespace

struct titan_ckpt {
    std::vector<std::unique_ptr<File>> files;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int> by_name;

    int add(Tensor&& t) {
        if (by_name.count(t.name)) return TITAN_ERR_IO;  // ambiguous name
        by_name[t.name] = (int)tensors.size();
        tensors.push_back(std::move(t));
        return TITAN_OK;
    }
    int open_file(const std::string& path) {
        auto f = std::make_unique<File>();
        f->fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (f->fd < 0) return -1;
        struct stat st;
        if (fstat(f->fd, &st) != 0) return -1;
        f->size = (uint64_t)st.st_size;
        files.push_back(std::move(f));
        return (int)files.size() - 1;
    }

    // safetensors: u64 header length, JSON header, data (loader.cpp:36-138, 166-196)
    int load_safetensors(const std::string& path) {
        const int fi = open_file(path);
        if (fi < 0) return TITAN_ERR_IO;
        const File& f = *files[fi];
        uint64_t hlen;
        if (!read_at(f, 0, &hlen, 8) || hlen > f.size - 8 || hlen > (256u << 20)) return TITAN_ERR_IO;
        std::string hdr((size_t)hlen, '\0');
        if (!read_at(f, 8, &hdr[0], hlen)) return TITAN_ERR_IO;
        JV root;
        if (!parse_json(hdr, root) || root.kind != JV::OBJ) return TITAN_ERR_IO;
        const uint64_t base = 8 + hlen;
        for (auto& kv : root.o) {
            if (kv.first == "__metadata__") continue;
            const JV& e = kv.second;
            const JV* dt = e.get("dtype");
            const JV* sh = e.get("shape");
            const JV* of = e.get("data_offsets");
            if (!dt || dt->kind != JV::STR || !sh || sh->kind != JV::ARR || !of || of->kind != JV::ARR ||
                of->a.size() != 2 || sh->a.size() > 8)
                return TITAN_ERR_IO;
            Tensor t;
            t.name = kv.first;
            t.dtype = st_dtype(dt->s);
            t.ndim = (int)sh->a.size();
            uint64_t numel = 1;
            for (int d = 0; d < t.ndim; d++) {
                uint64_t v;
                if (!as_u64(&sh->a[d], v)) return TITAN_ERR_IO;
                t.shape[d] = (int64_t)v;
                numel *= v;
            }
            uint64_t b, en;
            if (!as_u64(&of->a[0], b) || !as_u64(&of->a[1], en) || en < b || en > f.size - base)
                return TITAN_ERR_IO;
            t.file = fi;
            t.offset = base + b;
            t.nbytes = en - b;
            const int eb = ck_elem_bytes(t.dtype);
            if (eb && t.nbytes != numel * (uint64_t)eb) return TITAN_ERR_IO;
            if (int st = add(std::move(t))) return st;
        }
        return TITAN_OK;
    }

    // GGUF v2/v3 (gguf_loader.cpp:60-240): header, key/values (only
    // general.alignment is used), tensor infos, data at the next alignment.
    int load_gguf(const std::string& path) {
        const int fi = open_file(path);
        if (fi < 0) return TITAN_ERR_IO;
        const File& f = *files[fi];
        uint64_t pos = 0;
        bool bad = false;
        auto rd = [&](void* dst, uint64_t n) {
            if (bad || !read_at(f, pos, dst, n)) { bad = true; return; }
            pos += n;
        };
        auto u32 = [&]() { uint32_t v = 0; rd(&v, 4); return v; };
        auto u64 = [&]() { uint64_t v = 0; rd(&v, 8); return v; };
        auto gstr = [&](std::string* out) {
            uint64_t n = u64();
            if (bad || n > (1u << 24)) { bad = true; return; }
            if (out) {
                out->assign((size_t)n, '\0');
                rd(&(*out)[0], n);
            } else {
                pos += n;
            }
        };
        char magic[4];
        rd(magic, 4);
        if (bad || memcmp(magic, "GGUF", 4)) return TITAN_ERR_IO;
        const uint32_t version = u32();
        if (version < 2 || version > 3) return TITAN_ERR_UNSUPPORTED;
        const uint64_t ntensors = u64(), nkv = u64();
        if (bad || ntensors > (1u << 24) || nkv > (1u << 24)) return TITAN_ERR_IO;
        uint64_t alignment = 32;
        // scalar sizes of the GGUF value types 0..12 (8 string, 9 array: 0)
        static const int vsz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        std::function<void(uint32_t, uint64_t*)> skip_value = [&](uint32_t type, uint64_t* num) {
            if (bad) return;
            if (type == 8) {
                gstr(nullptr);
            } else if (type == 9) {
                const uint32_t et = u32();
                const uint64_t n = u64();
                if (bad || et > 12) { bad = true; return; }
                if (et == 8 || et == 9) {
                    for (uint64_t k = 0; k < n && !bad; k++) skip_value(et, nullptr);
                } else {
                    if (n > f.size) { bad = true; return; }
                    pos += n * (uint64_t)vsz[et];
                }
            } else if (type <= 12) {
                uint64_t v = 0;
                rd(&v, (uint64_t)vsz[type]);
                if (num) *num = v;
            } else {
                bad = true;
            }
        };
        for (uint64_t k = 0; k < nkv && !bad; k++) {
            std::string key;
            gstr(&key);
            const uint32_t type = u32();
            uint64_t v = 0;
            skip_value(type, &v);
            if (!bad && key == "general.alignment" && (type == 4 || type == 10) && v) alignment = v;
        }
        if (bad || (alignment & (alignment - 1))) return TITAN_ERR_IO;
        std::vector<Tensor> ts;
        for (uint64_t k = 0; k < ntensors && !bad; k++) {
            Tensor t;
            gstr(&t.name);
            const uint32_t nd = u32();
            if (bad || nd == 0 || nd > 8) return TITAN_ERR_IO;
            uint64_t ne[8], numel = 1;
            for (uint32_t d = 0; d < nd; d++) {
                ne[d] = u64();
                numel *= ne[d];
            }
            const uint32_t type = u32();
            t.offset = u64();
            if (bad) return TITAN_ERR_IO;
            t.ndim = (int)nd;
            for (uint32_t d = 0; d < nd; d++) t.shape[d] = (int64_t)ne[nd - 1 - d];  // outermost first
            t.ggml_type = (int)type;
            t.dtype = ggml_plain_dtype(type);
            int blk, bytes;
            if (!ggml_geometry(type, blk, bytes) || numel % (uint64_t)blk) return TITAN_ERR_UNSUPPORTED;
            t.nbytes = numel / (uint64_t)blk * (uint64_t)bytes;
            t.file = fi;
            ts.push_back(std::move(t));
        }
        if (bad) return TITAN_ERR_IO;
        const uint64_t data = (pos + alignment - 1) & ~(alignment - 1);
        for (auto& t : ts) {
            if (t.offset > f.size || data > f.size - t.offset || t.nbytes > f.size - data - t.offset)
                return TITAN_ERR_IO;
            t.offset += data;
            if (int st = add(std::move(t))) return st;
        }
        return TITAN_OK;
    }

    // titan-v1 (convert_titan.py:146-235): manifest.json lists, per .bin file,
    // entries {name, offset, size, dtype "int4" | "fp16", shape, group_size};
    // an int4 entry is int32 codes [rows][cols/8] | fp16 scales | fp16 biases
    // ([rows][cols/group_size] each).
    int load_titan_v1(const std::string& dir) {
        File mf;
        mf.fd = open((dir + "/manifest.json").c_str(), O_RDONLY | O_CLOEXEC);
        if (mf.fd < 0) return TITAN_ERR_IO;
        struct stat st;
        if (fstat(mf.fd, &st) != 0 || st.st_size > (64 << 20)) return TITAN_ERR_IO;
        mf.size = (uint64_t)st.st_size;
        std::string text((size_t)mf.size, '\0');
        if (!read_at(mf, 0, &text[0], mf.size)) return TITAN_ERR_IO;
        JV root;
        if (!parse_json(text, root) || root.kind != JV::OBJ) return TITAN_ERR_IO;
        const JV* fmt = root.get("format");
        if (!fmt || fmt->kind != JV::STR || fmt->s != "titan-v1") return TITAN_ERR_UNSUPPORTED;
        std::vector<const JV*> groups;
        for (const char* sec : {"files", "expert_index"}) {
            const JV* s = root.get(sec);
            if (s && s->kind == JV::OBJ)
                for (auto& kv : s->o) groups.push_back(&kv.second);
        }
        for (const JV* g : groups) {
            const JV* file = g->get("file");
            const JV* list = g->get("tensors");
            if (!file || file->kind != JV::STR || !list || list->kind != JV::ARR) return TITAN_ERR_IO;
            const int fi = open_file(dir + "/" + file->s);
            if (fi < 0) return TITAN_ERR_IO;
            const File& f = *files[fi];
            for (const JV& e : list->a) {
                const JV* nm = e.get("name");
                const JV* dt = e.get("dtype");
                const JV* sh = e.get("shape");
                uint64_t off, size;
                if (!nm || nm->kind != JV::STR || !dt || dt->kind != JV::STR || !sh || sh->kind != JV::ARR ||
                    sh->a.size() > 8 || !as_u64(e.get("offset"), off) || !as_u64(e.get("size"), size) ||
                    off > f.size || size > f.size - off)
                    return TITAN_ERR_IO;
                Tensor t;
                t.name = nm->s;
                t.ndim = (int)sh->a.size();
                uint64_t numel = 1;
                for (int d = 0; d < t.ndim; d++) {
                    uint64_t v;
                    if (!as_u64(&sh->a[d], v)) return TITAN_ERR_IO;
                    t.shape[d] = (int64_t)v;
                    numel *= v;
                }
                t.file = fi;
                t.offset = off;
                t.nbytes = size;
                if (dt->s == "int4") {
                    uint64_t gs;
                    if (!as_u64(e.get("group_size"), gs) || gs == 0 || t.ndim != 2) return TITAN_ERR_IO;
                    const uint64_t rows = (uint64_t)t.shape[0], cols = (uint64_t)t.shape[1];
                    if (cols % 8 || cols % gs || size != rows * cols / 2 + 4 * rows * (cols / gs))
                        return TITAN_ERR_IO;
                    t.dtype = TITAN_CK_INT4_AFFINE;
                    t.group_size = (int)gs;
                } else if (dt->s == "fp16") {
                    if (size != numel * 2) return TITAN_ERR_IO;
                    t.dtype = TITAN_CK_F16;
                } else {
                    return TITAN_ERR_UNSUPPORTED;
                }
                if (int s2 = add(std::move(t))) return s2;
            }
        }
        return TITAN_OK;
    }

    int open_path(const std::string& path) {
        if (is_dir(path)) {
            if (is_file(path + "/manifest.json")) return load_titan_v1(path);
            // every *.safetensors of the directory: the shards named by
            // model.safetensors.index.json and any others present (loader.cpp:266-290)
            std::vector<std::string> names;
            if (DIR* d = opendir(path.c_str())) {
                while (dirent* de = readdir(d)) {
                    std::string n = de->d_name;
                    if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) names.push_back(n);
                }
                closedir(d);
            }
            if (names.empty()) return TITAN_ERR_IO;
            std::sort(names.begin(), names.end());
            for (auto& n : names)
                if (int st = load_safetensors(path + "/" + n)) return st;
            return TITAN_OK;
        }
        File probe;
        probe.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (probe.fd < 0) return TITAN_ERR_IO;
        struct stat st;
        if (fstat(probe.fd, &st) != 0) return TITAN_ERR_IO;
        probe.size = (uint64_t)st.st_size;
        char magic[4] = {0};
        if (!read_at(probe, 0, magic, 4)) return TITAN_ERR_IO;
        return memcmp(magic, "GGUF", 4) == 0 ? load_gguf(path) : load_safetensors(path);
    }

    int find(const std::string& n) const {
        auto it = by_name.find(n);
        return it == by_name.end() ? -1 : it->second;
    }
    bool read(int i, void* dst) const {
        const Tensor& t = tensors[i];
        return read_at(*files[t.file], t.offset, dst, t.nbytes);
    }
};

namespace {

// What `name` resolves to: a direct quantized tensor or an NVFP4 triple.
struct Plan {
    titan_ckpt_weight w{};
    int direct = -1;            // tensor index (K-quant / INT4)
    int nv_w = -1, nv_s = -1, nv_g = -1;
};

int plan_weight(const titan_ckpt* ck, const char* name, Plan& pl) {
    if (!ck || !name) return TITAN_ERR_INVALID_ARG;
    const std::string n = name;
    pl = Plan();
    pl.w.global_scale = 1.0f;
    const int i = ck->find(n);
    if (i >= 0) {
        const Tensor& t = ck->tensors[i];
        if (t.ndim != 2 || t.shape[0] <= 0 || t.shape[1] <= 0 || t.shape[0] > INT32_MAX || t.shape[1] > INT32_MAX)
            return TITAN_ERR_UNSUPPORTED;
        pl.w.rows = (int)t.shape[0];
        pl.w.cols = (int)t.shape[1];
        if (t.dtype == TITAN_CK_GGML && (t.ggml_type == 12 || t.ggml_type == 11)) {
            pl.w.format = t.ggml_type == 12 ? TITAN_Q4_K : TITAN_Q3_K;
        } else if (t.dtype == TITAN_CK_INT4_AFFINE) {
            pl.w.format = TITAN_INT4;
            pl.w.group_size = t.group_size;
        } else {
            return TITAN_ERR_UNSUPPORTED;
        }
        pl.direct = i;
    } else {
        // NVFP4 projection (moe.cpp:613-724)
        pl.nv_w = ck->find(n + ".weight");
        pl.nv_s = ck->find(n + ".weight_scale");
        pl.nv_g = ck->find(n + ".weight_scale_2");
        if (pl.nv_w < 0 || pl.nv_s < 0) return TITAN_ERR_NOT_FOUND;
        const Tensor& w = ck->tensors[pl.nv_w];
        const Tensor& s = ck->tensors[pl.nv_s];
        if ((w.dtype != TITAN_CK_U8 && w.dtype != TITAN_CK_I8) || w.ndim != 2 ||
            (s.dtype != TITAN_CK_F8_E4M3 && s.dtype != TITAN_CK_U8) || s.ndim != 2)
            return TITAN_ERR_UNSUPPORTED;
        const int64_t rows = w.shape[0], cols = 2 * w.shape[1];
        if (rows <= 0 || cols > INT32_MAX || rows > INT32_MAX || s.shape[0] != rows || s.shape[1] * 16 != cols)
            return TITAN_ERR_UNSUPPORTED;
        pl.w.format = TITAN_NVFP4;
        pl.w.rows = (int)rows;
        pl.w.cols = (int)cols;
        if (pl.nv_g >= 0) {
            // F32 scalar, or a BF16 scalar widened; any other size: 1.0 (moe.cpp:670-699)
            const Tensor& g = ck->tensors[pl.nv_g];
            if (g.nbytes == 4) {
                if (!ck->read(pl.nv_g, &pl.w.global_scale)) return TITAN_ERR_IO;
            } else if (g.nbytes == 2) {
                uint16_t h;
                if (!ck->read(pl.nv_g, &h)) return TITAN_ERR_IO;
                const uint32_t bits = (uint32_t)h << 16;
                memcpy(&pl.w.global_scale, &bits, 4);
            }
        }
    }
    pl.w.tiled_bytes = titan_tiled_bytes(pl.w.format, pl.w.rows, pl.w.cols, pl.w.group_size);
    return pl.w.tiled_bytes ? TITAN_OK : TITAN_ERR_UNSUPPORTED;
}

}  // namespace

extern "C" int titan_ckpt_open(const char* path, titan_ckpt** out) {
    if (!path || !out) return TITAN_ERR_INVALID_ARG;
    *out = nullptr;
    auto ck = std::make_unique<titan_ckpt>();
    if (int st = ck->open_path(path)) return st;
    *out = ck.release();
    return TITAN_OK;
}

extern "C" void titan_ckpt_close(titan_ckpt* ck) { delete ck; }

extern "C" int titan_ckpt_count(const titan_ckpt* ck) { return ck ? (int)ck->tensors.size() : 0; }

extern "C" int titan_ckpt_tensor_at(const titan_ckpt* ck, int index, titan_ckpt_tensor* out) {
    if (!ck || !out || index < 0 || index >= (int)ck->tensors.size()) return TITAN_ERR_INVALID_ARG;
    const Tensor& t = ck->tensors[index];
    out->name = t.name.c_str();
    out->dtype = t.dtype;
    out->ggml_type = t.ggml_type;
    out->ndim = t.ndim;
    for (int d = 0; d < 8; d++) out->shape[d] = d < t.ndim ? t.shape[d] : 0;
    out->nbytes = t.nbytes;
    out->group_size = t.group_size;
    return TITAN_OK;
}

extern "C" int titan_ckpt_find(const titan_ckpt* ck, const char* name) {
    return ck && name ? ck->find(name) : -1;
}

extern "C" int titan_ckpt_read(const titan_ckpt* ck, int index, void* dst, size_t dst_bytes) {
    if (!ck || !dst || index < 0 || index >= (int)ck->tensors.size()) return TITAN_ERR_INVALID_ARG;
    if (dst_bytes < ck->tensors[index].nbytes) return TITAN_ERR_INVALID_ARG;
    return ck->read(index, dst) ? TITAN_OK : TITAN_ERR_IO;
}

extern "C" int titan_ckpt_weight_info(const titan_ckpt* ck, const char* name, titan_ckpt_weight* out) {
    if (!out) return TITAN_ERR_INVALID_ARG;
    Plan pl;
    if (int st = plan_weight(ck, name, pl)) return st;
    *out = pl.w;
    return TITAN_OK;
}

extern "C" int titan_ckpt_load_tiled(const titan_ckpt* ck, const char* name, void* tiled, size_t tiled_bytes,
                                     titan_ckpt_weight* out) {
    if (!tiled) return TITAN_ERR_INVALID_ARG;
    Plan pl;
    if (int st = plan_weight(ck, name, pl)) return st;
    if (tiled_bytes < pl.w.tiled_bytes) return TITAN_ERR_INVALID_ARG;
    const titan_ckpt_weight& w = pl.w;
    int st = TITAN_OK;
    if (pl.direct >= 0) {
        const Tensor& t = ck->tensors[pl.direct];
        std::vector<uint8_t> raw(t.nbytes);
        if (!ck->read(pl.direct, raw.data())) return TITAN_ERR_IO;
        if (w.format == TITAN_INT4) {
            const size_t codes = (size_t)w.rows * w.cols / 2, sb = (size_t)w.rows * (w.cols / w.group_size) * 2;
            st = titan_repack_host(TITAN_INT4, w.rows, w.cols, w.group_size, raw.data(), raw.data() + codes,
                                   raw.data() + codes + sb, tiled, tiled_bytes);
        } else {
            st = titan_repack_host(w.format, w.rows, w.cols, 0, raw.data(), nullptr, nullptr, tiled, tiled_bytes);
        }
    } else {
        const Tensor& tw = ck->tensors[pl.nv_w];
        const Tensor& ts = ck->tensors[pl.nv_s];
        std::vector<uint8_t> codes(tw.nbytes), scales(ts.nbytes);
        if (!ck->read(pl.nv_w, codes.data()) || !ck->read(pl.nv_s, scales.data())) return TITAN_ERR_IO;
        st = titan_repack_host(TITAN_NVFP4, w.rows, w.cols, 0, codes.data(), scales.data(), nullptr, tiled,
                               tiled_bytes);
    }
    if (st) return st;
    if (out) *out = w;
    return TITAN_OK;
}

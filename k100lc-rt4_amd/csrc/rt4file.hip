// rt4file.hip -- RT4 weight files: the manifest JSON and the 256-byte-aligned
// weight file that the reference converter writes (tools/convert.c:338-381 for
// the regions, :546-560 for the manifest), opened the way the reference runtime
// does (RT4::load / RT4::upload, src/model.cpp:141-185): parse the manifest,
// memory-map the weight file read-only, hand out host pointers into the
// mapping, and copy tensors (or the whole file) to the device.
//
// Manifest: {"format": "RT4-v1", "group": 128, "weight_file": "<path>",
// "tensors": [{"name", "kind", "shape": [..], "group", "q_off", "s_off",
// "nbytes", "relerr", "src_rms"}, ...]}.  Unlike the reference's substring scan,
// the manifest is parsed as JSON, and every tensor's regions are checked to lie
// inside the weight file before any pointer is handed out.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "rt4_internal.h"
#include "rt4k.h"

namespace {

int err(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return rt4::set_error(code, buf);
}

// ------------------------------------------------------------ JSON subset --
// Values of the manifest: objects, arrays, strings, numbers, true/false/null.
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    long long inum = 0;
    bool is_int = false;
    std::string str;
    std::vector<JVal> items;
    std::vector<std::pair<std::string, JVal>> fields;
    const JVal* get(const char* key) const {
        for (const auto& f : fields)
            if (f.first == key) return &f.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* end;
    std::string error;
    void ws() {
        while (p < end && isspace((unsigned char)*p)) p++;
    }
    bool fail(const char* what) {
        if (error.empty()) error = what;
        return false;
    }
    bool parse_string(std::string& out) {
        if (p >= end || *p != '"') return fail("expected a string");
        p++;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                if (++p >= end) return fail("bad escape");
                switch (*p) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'n': out += '\n'; break;
                    case 't': out += '\t'; break;
                    case 'r': out += '\r'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u': {  // kept as UTF-8 for the basic multilingual plane
                        if (end - p < 5) return fail("bad \\u escape");
                        char hex[5] = {p[1], p[2], p[3], p[4], 0};
                        const unsigned cp = (unsigned)strtoul(hex, nullptr, 16);
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xC0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3F));
                        } else {
                            out += (char)(0xE0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3F));
                            out += (char)(0x80 | (cp & 0x3F));
                        }
                        p += 4;
                        break;
                    }
                    default: return fail("bad escape");
                }
                p++;
            } else {
                out += *p++;
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool parse(JVal& v, int depth = 0) {
        if (depth > 32) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        const char c = *p;
        if (c == '{') {
            v.kind = JVal::OBJ;
            p++;
            ws();
            if (p < end && *p == '}') {
                p++;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!parse_string(key)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                p++;
                JVal val;
                if (!parse(val, depth + 1)) return false;
                v.fields.emplace_back(std::move(key), std::move(val));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == '}') {
                    p++;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = JVal::ARR;
            p++;
            ws();
            if (p < end && *p == ']') {
                p++;
                return true;
            }
            for (;;) {
                JVal val;
                if (!parse(val, depth + 1)) return false;
                v.items.push_back(std::move(val));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == ']') {
                    p++;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = JVal::STR;
            return parse_string(v.str);
        }
        if (!strncmp(p, "true", 4) || !strncmp(p, "false", 5)) {
            v.kind = JVal::BOOL;
            v.num = *p == 't';
            p += *p == 't' ? 4 : 5;
            return true;
        }
        if (!strncmp(p, "null", 4)) {
            p += 4;
            return true;
        }
        // number: integers are kept exact (offsets exceed 2^53 only for > 8 PB files)
        const char* q = p;
        if (q < end && (*q == '-' || *q == '+')) q++;
        bool frac = false;
        while (q < end && (isdigit((unsigned char)*q) || *q == '.' || *q == 'e' || *q == 'E' || *q == '-' || *q == '+')) {
            if (*q == '.' || *q == 'e' || *q == 'E') frac = true;
            q++;
        }
        if (q == p) return fail("unexpected character");
        const std::string tok(p, q);
        v.kind = JVal::NUM;
        v.num = strtod(tok.c_str(), nullptr);
        v.is_int = !frac;
        v.inum = frac ? (long long)v.num : strtoll(tok.c_str(), nullptr, 10);
        p = q;
        return true;
    }
};

// ------------------------------------------------------------------ file --
struct Tensor {
    std::string name, kind;
    int ndim = 0;
    int64_t shape[4] = {0, 0, 0, 0};
    int64_t group = 0, q_off = 0, s_off = -1, nbytes = 0;
    double relerr = 0, src_rms = 0;
    size_t q_bytes = 0, s_bytes = 0;  // sizes of the two regions
};

struct File {
    std::vector<Tensor> tensors;
    std::string weight_path;
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
};

bool as_i64(const JVal* v, int64_t* out) {
    if (!v || v->kind != JVal::NUM) return false;
    *out = v->is_int ? v->inum : (int64_t)v->num;
    return true;
}

std::string dir_of(const std::string& path) {
    const size_t s = path.rfind('/');
    return s == std::string::npos ? std::string(".") : path.substr(0, s);
}

// Region sizes of one tensor as the converter writes them (tools/convert.c:
// 338-377): "i4" = N*K/2 code bytes + N*(K/group) fp16 scales; "i8" = N*K code
// bytes + the same scales; other kinds (f16, f32, ...) are stored as-is,
// `nbytes` long, at q_off.
int sizes(const Tensor& t, size_t* q, size_t* s) {
    if (t.kind == "i4" || t.kind == "i8") {
        if (t.ndim != 2 || t.shape[0] <= 0 || t.shape[1] <= 0 || t.group <= 0 || t.shape[1] % t.group)
            return err(RT4_E_SHAPE, "rt4 file: tensor %s (%s): shape/group not a 2-D [N, K] with K %% group == 0",
                       t.name.c_str(), t.kind.c_str());
        const int64_t N = t.shape[0], K = t.shape[1];
        if (t.kind == "i4" && (K & 1))
            return err(RT4_E_SHAPE, "rt4 file: tensor %s: odd K for i4", t.name.c_str());
        *q = (size_t)(t.kind == "i4" ? N * K / 2 : N * K);
        *s = (size_t)(N * (K / t.group) * 2);
        return RT4_OK;
    }
    if (t.nbytes < 0) return err(RT4_E_SHAPE, "rt4 file: tensor %s: negative nbytes", t.name.c_str());
    *q = (size_t)t.nbytes;
    *s = 0;
    return RT4_OK;
}

int parse_manifest(const std::string& text, const std::string& manifest_path, File* f) {
    JParser jp{text.data(), text.data() + text.size(), {}};
    JVal root;
    if (!jp.parse(root)) return err(RT4_E_ARG, "rt4 file %s: manifest is not JSON (%s)", manifest_path.c_str(),
                                    jp.error.c_str());
    if (root.kind != JVal::OBJ) return err(RT4_E_ARG, "rt4 file %s: manifest is not an object", manifest_path.c_str());
    const JVal* fmt = root.get("format");
    if (fmt && (fmt->kind != JVal::STR || fmt->str != "RT4-v1"))
        return err(RT4_E_ARG, "rt4 file %s: unknown format", manifest_path.c_str());
    const JVal* wf = root.get("weight_file");
    if (wf && wf->kind == JVal::STR) f->weight_path = wf->str;
    int64_t group_default = 128;
    as_i64(root.get("group"), &group_default);
    const JVal* ts = root.get("tensors");
    if (!ts || ts->kind != JVal::ARR) return err(RT4_E_ARG, "rt4 file %s: no tensors array", manifest_path.c_str());
    for (const JVal& e : ts->items) {
        if (e.kind != JVal::OBJ) return err(RT4_E_ARG, "rt4 file %s: tensor entry is not an object", manifest_path.c_str());
        Tensor t;
        const JVal* name = e.get("name");
        const JVal* kind = e.get("kind");
        const JVal* shape = e.get("shape");
        if (!name || name->kind != JVal::STR || !kind || kind->kind != JVal::STR || !shape || shape->kind != JVal::ARR)
            return err(RT4_E_ARG, "rt4 file %s: tensor entry lacks name/kind/shape", manifest_path.c_str());
        t.name = name->str;
        t.kind = kind->str;
        if (shape->items.size() > 4) return err(RT4_E_SHAPE, "rt4 file: tensor %s has more than 4 dims", t.name.c_str());
        t.ndim = (int)shape->items.size();
        for (int d = 0; d < t.ndim; d++)
            if (!as_i64(&shape->items[d], &t.shape[d]) || t.shape[d] < 0)
                return err(RT4_E_SHAPE, "rt4 file: tensor %s: bad shape", t.name.c_str());
        t.group = group_default;
        as_i64(e.get("group"), &t.group);
        if (!as_i64(e.get("q_off"), &t.q_off) || t.q_off < 0)
            return err(RT4_E_ARG, "rt4 file: tensor %s: missing q_off", t.name.c_str());
        as_i64(e.get("s_off"), &t.s_off);
        as_i64(e.get("nbytes"), &t.nbytes);
        const JVal* v = e.get("relerr");
        if (v && v->kind == JVal::NUM) t.relerr = v->num;
        v = e.get("src_rms");
        if (v && v->kind == JVal::NUM) t.src_rms = v->num;
        int rc = sizes(t, &t.q_bytes, &t.s_bytes);
        if (rc) return rc;
        f->tensors.push_back(std::move(t));
    }
    return RT4_OK;
}

int check_regions(const File& f) {
    for (const Tensor& t : f.tensors) {
        if ((size_t)t.q_off > f.size || t.q_bytes > f.size - (size_t)t.q_off)
            return err(RT4_E_SHAPE, "rt4 file: tensor %s: code region [%lld, +%zu) outside the %zu-byte file",
                       t.name.c_str(), (long long)t.q_off, t.q_bytes, f.size);
        if (t.s_bytes) {
            if (t.s_off < 0 || (size_t)t.s_off > f.size || t.s_bytes > f.size - (size_t)t.s_off)
                return err(RT4_E_SHAPE, "rt4 file: tensor %s: scale region outside the file", t.name.c_str());
            if ((t.q_off | t.s_off) & 255)
                return err(RT4_E_SHAPE, "rt4 file: tensor %s: regions not 256-byte aligned", t.name.c_str());
        }
    }
    return RT4_OK;
}

File* as_file(void* h) { return static_cast<File*>(h); }

int check_index(File* f, int i, const char* who) {
    if (!f) return err(RT4_E_ARG, "%s: null file", who);
    if (i < 0 || i >= (int)f->tensors.size()) return err(RT4_E_ARG, "%s: tensor index %d out of range", who, i);
    return RT4_OK;
}

}  // namespace

extern "C" {

int rt4_file_open(const char* manifest_path, const char* weight_path, void** file) {
    if (!manifest_path || !file) return err(RT4_E_ARG, "rt4_file_open: null pointer");
    *file = nullptr;
    FILE* mf = fopen(manifest_path, "rb");
    if (!mf) return err(RT4_E_ARG, "rt4_file_open: cannot open %s", manifest_path);
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), mf)) > 0) text.append(buf, n);
    fclose(mf);
    File* f = new File;
    int rc = parse_manifest(text, manifest_path, f);
    if (rc) {
        delete f;
        return rc;
    }
    std::string wp = weight_path ? std::string(weight_path) : f->weight_path;
    if (wp.empty()) {
        delete f;
        return err(RT4_E_ARG, "rt4_file_open: %s names no weight file", manifest_path);
    }
    // a relative weight_file is tried as given, then next to the manifest
    int fd = open(wp.c_str(), O_RDONLY);
    if (fd < 0 && !weight_path && wp[0] != '/') {
        const size_t s = wp.rfind('/');
        const std::string alt = dir_of(manifest_path) + "/" + (s == std::string::npos ? wp : wp.substr(s + 1));
        fd = open(alt.c_str(), O_RDONLY);
        if (fd >= 0) wp = alt;
    }
    if (fd < 0) {
        delete f;
        return err(RT4_E_ARG, "rt4_file_open: cannot open weight file %s", wp.c_str());
    }
    struct stat st {};
    if (fstat(fd, &st) != 0) {
        close(fd);
        delete f;
        return err(RT4_E_ARG, "rt4_file_open: cannot stat %s", wp.c_str());
    }
    f->fd = fd;
    f->size = (size_t)st.st_size;
    f->weight_path = wp;
    if (f->size) {
        void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            delete f;
            return err(RT4_E_ARG, "rt4_file_open: mmap of %s failed", wp.c_str());
        }
        f->map = static_cast<const uint8_t*>(m);
    }
    if ((rc = check_regions(*f))) {
        rt4_file_close(f);
        return rc;
    }
    *file = f;
    return RT4_OK;
}

int rt4_file_close(void* file) {
    File* f = as_file(file);
    if (!f) return RT4_OK;
    if (f->map) munmap(const_cast<uint8_t*>(f->map), f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
    return RT4_OK;
}

int rt4_file_count(void* file, int* count) {
    File* f = as_file(file);
    if (!f || !count) return err(RT4_E_ARG, "rt4_file_count: null pointer");
    *count = (int)f->tensors.size();
    return RT4_OK;
}

int rt4_file_find(void* file, const char* name, int* index) {
    File* f = as_file(file);
    if (!f || !name || !index) return err(RT4_E_ARG, "rt4_file_find: null pointer");
    for (size_t i = 0; i < f->tensors.size(); i++)
        if (f->tensors[i].name == name) {
            *index = (int)i;
            return RT4_OK;
        }
    return err(RT4_E_ARG, "rt4_file_find: no tensor named %s", name);
}

int rt4_file_info(void* file, int index, rt4_tensor_info* info) {
    File* f = as_file(file);
    int rc = check_index(f, index, "rt4_file_info");
    if (rc) return rc;
    if (!info) return err(RT4_E_ARG, "rt4_file_info: null pointer");
    const Tensor& t = f->tensors[index];
    memset(info, 0, sizeof(*info));
    info->name = t.name.c_str();
    snprintf(info->kind, sizeof(info->kind), "%s", t.kind.c_str());
    info->ndim = t.ndim;
    for (int d = 0; d < 4; d++) info->shape[d] = t.shape[d];
    info->group = t.group;
    info->q_off = t.q_off;
    info->s_off = t.s_bytes ? t.s_off : -1;
    info->q_bytes = (int64_t)t.q_bytes;
    info->s_bytes = (int64_t)t.s_bytes;
    info->relerr = t.relerr;
    info->src_rms = t.src_rms;
    return RT4_OK;
}

int rt4_file_data(void* file, int index, const void** q, const void** s) {
    File* f = as_file(file);
    int rc = check_index(f, index, "rt4_file_data");
    if (rc) return rc;
    const Tensor& t = f->tensors[index];
    if (q) *q = f->map + t.q_off;
    if (s) *s = t.s_bytes ? f->map + t.s_off : nullptr;
    return RT4_OK;
}

int rt4_file_size(void* file, int64_t* bytes) {
    File* f = as_file(file);
    if (!f || !bytes) return err(RT4_E_ARG, "rt4_file_size: null pointer");
    *bytes = (int64_t)f->size;
    return RT4_OK;
}

int rt4_file_upload(void* file, void* dev, int64_t dev_bytes, void* stream) {
    File* f = as_file(file);
    if (!f || !dev) return err(RT4_E_ARG, "rt4_file_upload: null pointer");
    if (dev_bytes < (int64_t)f->size)
        return err(RT4_E_ARG, "rt4_file_upload: %lld-byte buffer for a %zu-byte file", (long long)dev_bytes, f->size);
    // 256 MB pieces from the pageable mapping, as the reference does (src/model.cpp:178-184)
    const size_t CH = (size_t)256 << 20;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for (size_t off = 0; off < f->size; off += CH) {
        const size_t n = f->size - off < CH ? f->size - off : CH;
        const hipError_t e = hipMemcpyAsync(static_cast<uint8_t*>(dev) + off, f->map + off, n, hipMemcpyHostToDevice, st);
        if (e != hipSuccess) return err(RT4_E_HIP, "rt4_file_upload: %s", hipGetErrorString(e));
    }
    const hipError_t e = hipStreamSynchronize(st);  // the mapping is pageable: finish before returning
    return e == hipSuccess ? RT4_OK : err(RT4_E_HIP, "rt4_file_upload: %s", hipGetErrorString(e));
}

int rt4_file_upload_tensor(void* file, int index, void* q_dev, void* s_dev, void* stream) {
    File* f = as_file(file);
    int rc = check_index(f, index, "rt4_file_upload_tensor");
    if (rc) return rc;
    const Tensor& t = f->tensors[index];
    if (!q_dev || (t.s_bytes && !s_dev)) return err(RT4_E_ARG, "rt4_file_upload_tensor: null pointer");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(q_dev, f->map + t.q_off, t.q_bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess && t.s_bytes) e = hipMemcpyAsync(s_dev, f->map + t.s_off, t.s_bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? RT4_OK : err(RT4_E_HIP, "rt4_file_upload_tensor %s: %s", t.name.c_str(), hipGetErrorString(e));
}

}  // extern "C"

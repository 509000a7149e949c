// GGUF file reader (host code): maps a .gguf file read-only, parses the header, the metadata
// key/value pairs and the tensor infos, and hands a tensor's blocks straight to
// uploadQuantized. This is the step before the quantized-matmul path: the reference takes
// its blobs from an external caller (core/tensor/QuantType.java:3 names the GGUF type ids;
// spi/QuantizedOps.java:24 takes the blob).
//
// Layout (GGUF v2/v3, little-endian): magic "GGUF", u32 version, u64 tensor count, u64
// metadata count; metadata entries (string key, u32 value type, value); tensor infos (string
// name, u32 n_dims, u64 dims[n_dims] innermost first, u32 ggml type, u64 offset relative to
// the data section); the data section starts at the next multiple of general.alignment
// (default 32) and every tensor offset is a multiple of it. A string is a u64 length and
// that many bytes; an array is a u32 element type, a u64 count and the elements.
//
// The file is untrusted: every length, count and offset is checked against the mapping
// before it is read, and a failed check is J4Q_EINVAL with the byte position in the message.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "engine.h"

namespace {

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

int scalar_size(uint32_t t) {
    switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
    }
}

// Block geometry of the ggml type ids GGUF files carry (ids as in core/tensor/QuantType.java:5-13
// for the rows the reference knows, the remaining upstream ggml ids from the published format).
bool ggml_geometry(uint32_t id, int *elems, int *bytes) {
    switch (id) {
    case 0: *elems = 1; *bytes = 4; return true;      // F32
    case 1: *elems = 1; *bytes = 2; return true;      // F16
    case 2: *elems = 32; *bytes = 18; return true;    // Q4_0
    case 3: *elems = 32; *bytes = 20; return true;    // Q4_1
    case 6: *elems = 32; *bytes = 22; return true;    // Q5_0
    case 7: *elems = 32; *bytes = 24; return true;    // Q5_1
    case 8: *elems = 32; *bytes = 34; return true;    // Q8_0
    case 9: *elems = 32; *bytes = 36; return true;    // Q8_1
    case 10: *elems = 256; *bytes = 84; return true;  // Q2_K
    case 11: *elems = 256; *bytes = 110; return true; // Q3_K
    case 12: *elems = 256; *bytes = 144; return true; // Q4_K
    case 13: *elems = 256; *bytes = 176; return true; // Q5_K
    case 14: *elems = 256; *bytes = 210; return true; // Q6_K
    case 15: *elems = 256; *bytes = 292; return true; // Q8_K
    case 30: *elems = 1; *bytes = 2; return true;     // BF16
    case 41: *elems = 256; *bytes = 34; return true;  // Q1_0 (prism fork)
    case 42: *elems = 128; *bytes = 34; return true;  // Q2_0 (prism fork)
    default: return false;
    }
}

struct Meta {
    std::string key;
    uint32_t type = 0;
    uint64_t pos = 0;         // file offset of the value
    uint32_t elem_type = 0;   // arrays
    uint64_t count = 0;       // arrays: element count; strings: byte length
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0;  // absolute file offset
    uint64_t nbytes = 0;  // 0 if the type's geometry is unknown
};

struct File {
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    std::vector<Meta> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::string path;
};

std::mutex g_gmu;
std::vector<File *> g_files;  // handle = index + 1 (closed slots hold nullptr)

class Reader {
  public:
    Reader(const uint8_t *p, uint64_t n) : p_(p), n_(n) {}
    uint64_t pos() const { return off_; }
    bool need(uint64_t k) const { return k <= n_ && off_ <= n_ - k; }
    template <typename T>
    int get(T *v, const char *what) {
        if (!need(sizeof(T))) return j4q::report_error(J4Q_EINVAL, "GGUF: truncated reading %s at byte %llu", what, (unsigned long long)off_);
        memcpy(v, p_ + off_, sizeof(T));
        off_ += sizeof(T);
        return J4Q_OK;
    }
    int skip(uint64_t k, const char *what) {
        if (!need(k)) return j4q::report_error(J4Q_EINVAL, "GGUF: truncated %s at byte %llu", what, (unsigned long long)off_);
        off_ += k;
        return J4Q_OK;
    }
    int str(std::string *s, const char *what) {
        uint64_t len;
        int rc = get(&len, what);
        if (rc) return rc;
        if (len > (1u << 20) || !need(len))
            return j4q::report_error(J4Q_EINVAL, "GGUF: %s string of %llu bytes at byte %llu exceeds the file", what,
                                  (unsigned long long)len, (unsigned long long)off_);
        s->assign(reinterpret_cast<const char *>(p_ + off_), len);
        off_ += len;
        return J4Q_OK;
    }

  private:
    const uint8_t *p_;
    uint64_t n_, off_ = 0;
};

// Skips one metadata value of type t (arrays of arrays included, depth-limited).
int skip_value(Reader &r, uint32_t t, int depth) {
    if (depth > 4) return j4q::report_error(J4Q_EINVAL, "GGUF: arrays nested too deeply at byte %llu", (unsigned long long)r.pos());
    if (const int sz = scalar_size(t)) return r.skip((uint64_t)sz, "metadata value");
    if (t == T_STRING) {
        std::string s;
        return r.str(&s, "metadata");
    }
    if (t == T_ARRAY) {
        uint32_t et;
        uint64_t cnt;
        int rc = r.get(&et, "array type");
        if (!rc) rc = r.get(&cnt, "array count");
        if (rc) return rc;
        if (const int sz = scalar_size(et)) {
            if (cnt > (uint64_t)1 << 40) return j4q::report_error(J4Q_EINVAL, "GGUF: array of %llu elements", (unsigned long long)cnt);
            return r.skip(cnt * (uint64_t)sz, "array");
        }
        for (uint64_t i = 0; i < cnt; i++)
            if ((rc = skip_value(r, et, depth + 1))) return rc;
        return J4Q_OK;
    }
    return j4q::report_error(J4Q_EINVAL, "GGUF: unknown metadata value type %u at byte %llu", t, (unsigned long long)r.pos());
}

int parse(File *f) {
    Reader r(f->map, f->size);
    uint32_t magic;
    int rc = r.get(&magic, "magic");
    if (rc) return rc;
    if (magic != 0x46554747u) return j4q::report_error(J4Q_EINVAL, "GGUF: bad magic 0x%08x (not a GGUF file)", magic);
    if ((rc = r.get(&f->version, "version"))) return rc;
    if (f->version != 2 && f->version != 3)
        return j4q::report_error(J4Q_EUNSUPPORTED, "GGUF: version %u not supported (2 or 3)", f->version);
    uint64_t nt, nkv;
    if ((rc = r.get(&nt, "tensor count")) || (rc = r.get(&nkv, "metadata count"))) return rc;
    // every entry takes more than 8 bytes, so larger counts cannot fit the file
    if (nt > f->size / 8 || nkv > f->size / 8)
        return j4q::report_error(J4Q_EINVAL, "GGUF: %llu tensors / %llu metadata entries cannot fit %llu bytes",
                              (unsigned long long)nt, (unsigned long long)nkv, (unsigned long long)f->size);
    for (uint64_t i = 0; i < nkv; i++) {
        Meta m;
        if ((rc = r.str(&m.key, "metadata key")) || (rc = r.get(&m.type, "metadata type"))) return rc;
        m.pos = r.pos();
        if (m.type == T_ARRAY) {
            Reader peek = r;
            if ((rc = peek.get(&m.elem_type, "array type")) || (rc = peek.get(&m.count, "array count"))) return rc;
        } else if (m.type == T_STRING) {
            Reader peek = r;
            if ((rc = peek.get(&m.count, "string length"))) return rc;
        }
        if ((rc = skip_value(r, m.type, 0))) return rc;
        if (m.key == "general.alignment") {
            if (m.type != T_U32) return j4q::report_error(J4Q_EINVAL, "GGUF: general.alignment has type %u, not u32", m.type);
            uint32_t a;
            memcpy(&a, f->map + m.pos, 4);
            if (a == 0 || (a & (a - 1)) != 0) return j4q::report_error(J4Q_EINVAL, "GGUF: general.alignment %u is not a power of two", a);
            f->alignment = a;
        }
        f->meta.push_back(std::move(m));
    }
    for (uint64_t i = 0; i < nt; i++) {
        Tensor t;
        if ((rc = r.str(&t.name, "tensor name")) || (rc = r.get(&t.n_dims, "tensor n_dims"))) return rc;
        if (t.n_dims == 0 || t.n_dims > 4)
            return j4q::report_error(J4Q_EINVAL, "GGUF: tensor '%s' has %u dimensions (1..4)", t.name.c_str(), t.n_dims);
        uint64_t elems = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            if ((rc = r.get(&t.dims[d], "tensor dims"))) return rc;
            if (t.dims[d] == 0 || t.dims[d] > ((uint64_t)1 << 40) || elems > ((uint64_t)1 << 62) / t.dims[d])
                return j4q::report_error(J4Q_EINVAL, "GGUF: tensor '%s' dimension %u = %llu out of range", t.name.c_str(), d,
                                      (unsigned long long)t.dims[d]);
            elems *= t.dims[d];
        }
        if ((rc = r.get(&t.type, "tensor type")) || (rc = r.get(&t.offset, "tensor offset"))) return rc;
        int be, bb;
        if (ggml_geometry(t.type, &be, &bb)) {
            if (t.dims[0] % (uint64_t)be != 0)
                return j4q::report_error(J4Q_EINVAL, "GGUF: tensor '%s' row of %llu elements is not a multiple of its block (%d)",
                                      t.name.c_str(), (unsigned long long)t.dims[0], be);
            t.nbytes = elems / (uint64_t)be * (uint64_t)bb;
        }
        if (f->by_name.count(t.name)) return j4q::report_error(J4Q_EINVAL, "GGUF: duplicate tensor name '%s'", t.name.c_str());
        f->by_name[t.name] = f->tensors.size();
        f->tensors.push_back(std::move(t));
    }
    const uint64_t end = r.pos();
    f->data_offset = (end + f->alignment - 1) / f->alignment * f->alignment;
    for (Tensor &t : f->tensors) {
        if (t.offset % f->alignment != 0)
            return j4q::report_error(J4Q_EINVAL, "GGUF: tensor '%s' offset %llu is not a multiple of the alignment %llu",
                                  t.name.c_str(), (unsigned long long)t.offset, (unsigned long long)f->alignment);
        if (t.offset > f->size || f->data_offset > f->size - t.offset || t.nbytes > f->size - f->data_offset - t.offset)
            return j4q::report_error(J4Q_EINVAL, "GGUF: tensor '%s' (%llu bytes at data offset %llu) extends past the end of the file (%llu bytes)",
                                  t.name.c_str(), (unsigned long long)t.nbytes, (unsigned long long)t.offset, (unsigned long long)f->size);
        t.offset += f->data_offset;
    }
    return J4Q_OK;
}

// Requires g_gmu held.
File *file_of(j4q_gguf h) {
    if (h == 0 || h > g_files.size()) return nullptr;
    return g_files[h - 1];
}

int get_file(j4q_gguf h, File **f) {
    *f = file_of(h);
    return *f ? J4Q_OK : j4q::report_error(J4Q_EHANDLE, "GGUF: unknown or closed file handle %llu", (unsigned long long)h);
}

int get_tensor(File *f, int64_t index, Tensor **t) {
    if (index < 0 || (uint64_t)index >= f->tensors.size())
        return j4q::report_error(J4Q_EINVAL, "GGUF: tensor index %lld out of range [0, %zu)", (long long)index, f->tensors.size());
    *t = &f->tensors[(size_t)index];
    return J4Q_OK;
}

int get_meta(File *f, const char *key, Meta **m) {
    if (!key) return j4q::report_error(J4Q_EINVAL, "GGUF: key is NULL");
    for (Meta &e : f->meta)
        if (e.key == key) {
            *m = &e;
            return J4Q_OK;
        }
    return j4q::report_error(J4Q_EINVAL, "GGUF: no metadata key '%s'", key);
}

void copy_cstr(char *dst, size_t cap, const std::string &s) {
    if (!dst || cap == 0) return;
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    memcpy(dst, s.data(), n);
    dst[n] = 0;
}

}  // namespace

extern "C" {

int j4q_gguf_open(const char *path, j4q_gguf *out) {
    if (!path || !out) return j4q::report_error(J4Q_EINVAL, "GGUF: NULL argument");
    *out = 0;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return j4q::report_error(J4Q_EINVAL, "GGUF: cannot open '%s': %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return j4q::report_error(J4Q_EINVAL, "GGUF: '%s' is empty or unreadable", path);
    }
    void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return j4q::report_error(J4Q_ENOMEM, "GGUF: cannot map '%s': %s", path, strerror(errno));
    File *f = new File;
    f->map = static_cast<const uint8_t *>(map);
    f->size = (uint64_t)st.st_size;
    f->path = path;
    const int rc = parse(f);
    if (rc) {
        munmap(const_cast<uint8_t *>(f->map), f->size);
        delete f;
        return rc;
    }
    std::lock_guard<std::mutex> lk(g_gmu);
    g_files.push_back(f);
    *out = (j4q_gguf)g_files.size();
    return J4Q_OK;
}

int j4q_gguf_close(j4q_gguf h) {
    if (h == 0) return J4Q_OK;
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    if (int rc = get_file(h, &f)) return rc;
    munmap(const_cast<uint8_t *>(f->map), f->size);
    delete f;
    g_files[h - 1] = nullptr;
    return J4Q_OK;
}

int j4q_gguf_file_info(j4q_gguf h, j4q_gguf_info *out) {
    if (!out) return j4q::report_error(J4Q_EINVAL, "GGUF: out is NULL");
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    if (int rc = get_file(h, &f)) return rc;
    out->version = f->version;
    out->reserved = 0;
    out->tensor_count = (int64_t)f->tensors.size();
    out->metadata_count = (int64_t)f->meta.size();
    out->alignment = f->alignment;
    out->data_offset = f->data_offset;
    out->file_bytes = f->size;
    return J4Q_OK;
}

int j4q_gguf_tensor_info(j4q_gguf h, int64_t index, j4q_gguf_tensor *out) {
    if (!out) return j4q::report_error(J4Q_EINVAL, "GGUF: out is NULL");
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    Tensor *t;
    if (int rc = get_file(h, &f)) return rc;
    if (int rc = get_tensor(f, index, &t)) return rc;
    memset(out, 0, sizeof *out);
    copy_cstr(out->name, sizeof out->name, t->name);
    out->type_id = (int32_t)t->type;
    out->n_dims = (int32_t)t->n_dims;
    for (int d = 0; d < 4; d++) out->dims[d] = (int64_t)t->dims[d];
    out->offset = t->offset;
    out->nbytes = t->nbytes;
    return J4Q_OK;
}

int j4q_gguf_find_tensor(j4q_gguf h, const char *name, int64_t *index) {
    if (!name || !index) return j4q::report_error(J4Q_EINVAL, "GGUF: NULL argument");
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    if (int rc = get_file(h, &f)) return rc;
    const auto it = f->by_name.find(name);
    if (it == f->by_name.end()) return j4q::report_error(J4Q_EINVAL, "GGUF: no tensor named '%s'", name);
    *index = (int64_t)it->second;
    return J4Q_OK;
}

int j4q_gguf_meta_key(j4q_gguf h, int64_t index, char *key, int32_t cap, int32_t *type, int32_t *elem_type,
                      uint64_t *count) {
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    if (int rc = get_file(h, &f)) return rc;
    if (index < 0 || (uint64_t)index >= f->meta.size())
        return j4q::report_error(J4Q_EINVAL, "GGUF: metadata index %lld out of range [0, %zu)", (long long)index, f->meta.size());
    const Meta &m = f->meta[(size_t)index];
    if (cap > 0) copy_cstr(key, (size_t)cap, m.key);
    if (type) *type = (int32_t)m.type;
    if (elem_type) *elem_type = (int32_t)m.elem_type;
    if (count) *count = m.count;
    return J4Q_OK;
}

int j4q_gguf_meta_scalar(j4q_gguf h, const char *key, int32_t *type, void *value8) {
    if (!value8) return j4q::report_error(J4Q_EINVAL, "GGUF: value is NULL");
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    Meta *m;
    if (int rc = get_file(h, &f)) return rc;
    if (int rc = get_meta(f, key, &m)) return rc;
    const int sz = scalar_size(m->type);
    if (!sz) return j4q::report_error(J4Q_EINVAL, "GGUF: metadata '%s' has type %u, not a scalar", key, m->type);
    memset(value8, 0, 8);
    memcpy(value8, f->map + m->pos, (size_t)sz);
    if (type) *type = (int32_t)m->type;
    return J4Q_OK;
}

int j4q_gguf_meta_string(j4q_gguf h, const char *key, char *out, uint64_t cap, uint64_t *length) {
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    Meta *m;
    if (int rc = get_file(h, &f)) return rc;
    if (int rc = get_meta(f, key, &m)) return rc;
    if (m->type != T_STRING) return j4q::report_error(J4Q_EINVAL, "GGUF: metadata '%s' has type %u, not a string", key, m->type);
    if (length) *length = m->count;
    if (out && cap > 0) {
        const uint64_t n = m->count < cap - 1 ? m->count : cap - 1;
        memcpy(out, f->map + m->pos + 8, n);
        out[n] = 0;
    }
    return J4Q_OK;
}

int j4q_gguf_read_tensor(j4q_gguf h, int64_t index, void *dst, uint64_t nbytes) {
    if (!dst) return j4q::report_error(J4Q_EINVAL, "GGUF: dst is NULL");
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    Tensor *t;
    if (int rc = get_file(h, &f)) return rc;
    if (int rc = get_tensor(f, index, &t)) return rc;
    if (t->nbytes == 0) return j4q::report_error(J4Q_EUNSUPPORTED, "GGUF: tensor '%s' has ggml type %u of unknown size", t->name.c_str(), t->type);
    if (nbytes != t->nbytes)
        return j4q::report_error(J4Q_EINVAL, "GGUF: tensor '%s' holds %llu bytes, not %llu", t->name.c_str(),
                              (unsigned long long)t->nbytes, (unsigned long long)nbytes);
    memcpy(dst, f->map + t->offset, t->nbytes);
    return J4Q_OK;
}

int j4q_gguf_upload(j4q_gguf h, int64_t index, j4q_buffer *out) {
    if (!out) return j4q::report_error(J4Q_EINVAL, "GGUF: out is NULL");
    // The file lock is held through the upload, so a concurrent close cannot unmap the
    // blocks while they are copied (the engine lock is only ever taken after this one).
    std::lock_guard<std::mutex> lk(g_gmu);
    File *f;
    Tensor *t;
    if (int rc = get_file(h, &f)) return rc;
    if (int rc = get_tensor(f, index, &t)) return rc;
    // a matrix [rows, cols] is stored innermost first: dims[0] = cols, the rest are rows
    const int64_t cols = (int64_t)t->dims[0];
    const int64_t rows = (int64_t)(t->dims[1] * t->dims[2] * t->dims[3]);
    return j4q_upload_quantized((int)t->type, f->map + t->offset, t->nbytes, rows, cols, out);
}

}  // extern "C"

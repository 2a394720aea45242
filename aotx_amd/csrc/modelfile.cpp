/* GGUF model files: header, metadata, tensor table and tensor bytes (host only).
 *
 * Reference: disk/modelfile/modelfile.h (format and API), disk/modelfile/gguf.h (limits),
 * disk/modelfile/gguf.c:411-541 (open, read); behaviour pinned by tests/gguf_test.c.
 *
 * The head of the file (header, metadata pairs, tensor infos) is read once into memory,
 * parsed with a bounds-checked cursor, and released; every value the caller can ask for is
 * copied out of it, so nothing points into the head. Every count in the file is checked
 * against the bytes it would need before anything is allocated, and all allocations of one
 * file are charged against a fixed budget. Codes: 0 ran, 1 the file cannot be read,
 * 2 the format is wrong (the file is then not opened).
 */
#include "modelfile.h"

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <string>
#include <vector>

namespace {

struct Meta {
    std::string key;
    uint32_t type = 0;
    uint32_t element_type = 0;
    uint64_t count = 0;                 /* array elements */
    uint64_t u = 0;                     /* unsigned value (or the bits of a signed one) */
    int64_t i = 0;
    double f = 0.0;
    bool negative = false;
    std::string text;                   /* a string value */
    std::vector<uint8_t> run;           /* string array bytes, or bool array elements */
    std::vector<uint64_t> offsets;      /* string array: count + 1 entries into run */
    std::vector<int32_t> i32;
    std::vector<float> f32;
};

uint64_t type_size(uint32_t t)
{
    switch (t) {
    case AOTX_GGUF_U8: case AOTX_GGUF_I8: case AOTX_GGUF_BOOL: return 1;
    case AOTX_GGUF_U16: case AOTX_GGUF_I16: return 2;
    case AOTX_GGUF_U32: case AOTX_GGUF_I32: case AOTX_GGUF_F32: return 4;
    case AOTX_GGUF_U64: case AOTX_GGUF_I64: case AOTX_GGUF_F64: return 8;
    default: return 0;
    }
}

/* Weights per block and bytes per block of a tensor type; false for a type the system
 * does not stream (it may still appear in a file). */
bool tensor_block(uint32_t type, uint64_t *weights, uint64_t *bytes)
{
    switch (type) {
    case AOTX_TENSOR_F32: *weights = 1; *bytes = 4; return true;
    case AOTX_TENSOR_F16: *weights = 1; *bytes = 2; return true;
    case AOTX_TENSOR_Q4_0: *weights = 32; *bytes = 18; return true;
    case AOTX_TENSOR_Q4_1: *weights = 32; *bytes = 20; return true;
    case AOTX_TENSOR_Q5_0: *weights = 32; *bytes = 22; return true;
    case AOTX_TENSOR_Q5_1: *weights = 32; *bytes = 24; return true;
    case AOTX_TENSOR_Q8_0: *weights = 32; *bytes = 34; return true;
    case AOTX_TENSOR_Q2_K: *weights = 256; *bytes = 84; return true;
    case AOTX_TENSOR_Q3_K: *weights = 256; *bytes = 110; return true;
    case AOTX_TENSOR_Q4_K: *weights = 256; *bytes = 144; return true;
    case AOTX_TENSOR_Q5_K: *weights = 256; *bytes = 176; return true;
    case AOTX_TENSOR_Q6_K: *weights = 256; *bytes = 210; return true;
    default: return false;
    }
}

} // namespace

struct aotx_modelfile {
    int fd = -1;
    std::string path;
    uint64_t file_bytes = 0;
    uint64_t data_offset = 0;
    uint64_t data_bytes = 0;
    uint32_t alignment = AOTX_GGUF_ALIGN;
    std::vector<Meta> meta;
    std::vector<aotx_tensor_info> tensors;
    std::vector<bool> streams;          /* per tensor: a type whose bytes are known */
    /* parse state (released after open) */
    std::vector<uint8_t> head;
    uint64_t pos = 0;
    uint64_t charged = 0;
};

namespace {

int refuse(const aotx_modelfile *f, const char *why)
{
    fprintf(stderr, "aotx: the model file %s is refused: %s\n", f->path.c_str(), why);
    return 2;
}

int charge(aotx_modelfile *f, uint64_t bytes)
{
    if (bytes > AOTX_GGUF_MEMORY_LIMIT || f->charged + bytes > AOTX_GGUF_MEMORY_LIMIT)
        return refuse(f, "the metadata needs more memory than the bound");
    f->charged += bytes;
    return 0;
}

/* Make the head hold the file bytes [0, pos + bytes). */
int need(aotx_modelfile *f, uint64_t bytes)
{
    if (bytes > f->file_bytes || f->pos > f->file_bytes - bytes)
        return refuse(f, "a field runs past the end of the file");
    const uint64_t want = f->pos + bytes;
    if (want <= f->head.size()) return 0;
    if (want > AOTX_GGUF_HEAD_LIMIT) return refuse(f, "the head is longer than the bound");
    /* grow in steps of at least 1 MiB, never past the file or the bound */
    uint64_t grow = want - f->head.size();
    if (grow < (1u << 20)) grow = 1u << 20;
    uint64_t upto = f->head.size() + grow;
    if (upto > f->file_bytes) upto = f->file_bytes;
    if (upto > AOTX_GGUF_HEAD_LIMIT) upto = AOTX_GGUF_HEAD_LIMIT;
    if (charge(f, upto - f->head.size()) != 0) return 2;
    const uint64_t have = f->head.size();
    try {
        f->head.resize(upto);
    } catch (const std::bad_alloc &) {
        return refuse(f, "the head does not fit in memory");
    }
    uint64_t at = have;
    while (at < upto) {
        ssize_t got = pread(f->fd, f->head.data() + at, (size_t)(upto - at), (off_t)at);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return refuse(f, "the file ends inside its head");
        at += (uint64_t)got;
    }
    return 0;
}

int number(aotx_modelfile *f, unsigned width, uint64_t *out)
{
    if (need(f, width) != 0) return 2;
    uint64_t v = 0;
    for (unsigned b = 0; b < width; ++b) v |= (uint64_t)f->head[f->pos + b] << (8u * b);
    f->pos += width;
    *out = v;
    return 0;
}

/* A string: an 8-byte length, then its bytes (left in the head). */
int string_at(aotx_modelfile *f, uint64_t *at, uint64_t *len)
{
    if (number(f, 8, len) != 0 || need(f, *len) != 0) return 2;
    *at = f->pos;
    f->pos += *len;
    return 0;
}

int scalar(aotx_modelfile *f, uint32_t type, Meta *m)
{
    const uint64_t w = type_size(type);
    uint64_t v = 0;
    if (number(f, (unsigned)w, &v) != 0) return 2;
    switch (type) {
    case AOTX_GGUF_BOOL:
        if (v > 1u) return refuse(f, "a boolean value is neither 0 nor 1");
        m->u = v;
        break;
    case AOTX_GGUF_I8: m->i = (int8_t)v; break;
    case AOTX_GGUF_I16: m->i = (int16_t)v; break;
    case AOTX_GGUF_I32: m->i = (int32_t)v; break;
    case AOTX_GGUF_I64: m->i = (int64_t)v; break;
    case AOTX_GGUF_F32: {
        uint32_t b = (uint32_t)v;
        float x;
        memcpy(&x, &b, 4);
        m->f = x;
        break;
    }
    case AOTX_GGUF_F64: memcpy(&m->f, &v, 8); break;
    default: m->u = v; break;
    }
    if (type == AOTX_GGUF_I8 || type == AOTX_GGUF_I16 || type == AOTX_GGUF_I32 || type == AOTX_GGUF_I64) {
        m->negative = m->i < 0;
        m->u = (uint64_t)m->i;
    }
    return 0;
}

int value(aotx_modelfile *f, Meta *m)
{
    uint64_t t = 0;
    if (number(f, 4, &t) != 0) return 2;
    m->type = (uint32_t)t;
    if (m->type == AOTX_GGUF_STRING) {
        uint64_t at = 0, len = 0;
        if (string_at(f, &at, &len) != 0 || charge(f, len + 1) != 0) return 2;
        m->text.assign((const char *)f->head.data() + at, (size_t)len);
        return 0;
    }
    if (m->type != AOTX_GGUF_ARRAY) {
        if (type_size(m->type) == 0) return refuse(f, "a metadata value has an unknown type");
        return scalar(f, m->type, m);
    }
    uint64_t et = 0, count = 0;
    if (number(f, 4, &et) != 0 || number(f, 8, &count) != 0) return 2;
    m->element_type = (uint32_t)et;
    m->count = count;
    if (m->element_type == AOTX_GGUF_ARRAY) return refuse(f, "an array holds arrays");
    if (m->element_type == AOTX_GGUF_STRING) {
        /* each element holds at least its 8-byte length */
        if (count > (f->file_bytes - f->pos) / 8u) return refuse(f, "an array count runs past the end");
        if (charge(f, (count + 1u) * 8u) != 0) return 2;
        m->offsets.assign((size_t)count + 1u, 0u);
        for (uint64_t e = 0; e < count; ++e) {
            uint64_t at = 0, len = 0;
            if (string_at(f, &at, &len) != 0 || charge(f, len) != 0) return 2;
            m->run.insert(m->run.end(), f->head.begin() + (ptrdiff_t)at,
                          f->head.begin() + (ptrdiff_t)(at + len));
            m->offsets[(size_t)e + 1u] = m->run.size();
        }
        return 0;
    }
    const uint64_t w = type_size(m->element_type);
    if (w == 0) return refuse(f, "an array element has an unknown type");
    if (count > (f->file_bytes - f->pos) / w) return refuse(f, "an array count runs past the end");
    if (need(f, count * w) != 0) return 2;
    const uint8_t *p = f->head.data() + f->pos;
    if (m->element_type == AOTX_GGUF_I32) {
        if (charge(f, count * 4u) != 0) return 2;
        m->i32.resize((size_t)count);
        memcpy(m->i32.data(), p, (size_t)count * 4u);
    } else if (m->element_type == AOTX_GGUF_F32) {
        if (charge(f, count * 4u) != 0) return 2;
        m->f32.resize((size_t)count);
        memcpy(m->f32.data(), p, (size_t)count * 4u);
    } else if (m->element_type == AOTX_GGUF_BOOL) {
        if (charge(f, count) != 0) return 2;
        for (uint64_t e = 0; e < count; ++e)
            if (p[e] > 1u) return refuse(f, "a boolean element is neither 0 nor 1");
        m->run.assign(p, p + count);
    }
    /* other element types are checked and skipped: no getter gives them */
    f->pos += count * w;
    return 0;
}

int parse(aotx_modelfile *f)
{
    uint64_t magic = 0, version = 0, tensors = 0, pairs = 0;
    if (number(f, 4, &magic) != 0 || number(f, 4, &version) != 0) return 2;
    if (magic != AOTX_GGUF_MAGIC) return refuse(f, "the magic is not GGUF");
    if (version != AOTX_GGUF_VERSION) return refuse(f, "the version is not 3");
    if (number(f, 8, &tensors) != 0 || number(f, 8, &pairs) != 0) return 2;
    const uint64_t rest = f->file_bytes - f->pos;
    if (pairs > rest / AOTX_GGUF_PAIR_LEAST) return refuse(f, "the metadata count exceeds the file");
    if (tensors > rest / AOTX_GGUF_TENSOR_LEAST) return refuse(f, "the tensor count exceeds the file");
    if (charge(f, pairs * sizeof(Meta) + tensors * (sizeof(aotx_tensor_info) + 1u)) != 0) return 2;
    f->meta.resize((size_t)pairs);
    bool have_align = false;
    for (uint64_t i = 0; i < pairs; ++i) {
        Meta &m = f->meta[(size_t)i];
        uint64_t at = 0, len = 0;
        if (string_at(f, &at, &len) != 0) return 2;
        if (len == 0 || len >= AOTX_GGUF_KEY_BYTES) return refuse(f, "a metadata key is empty or too long");
        m.key.assign((const char *)f->head.data() + at, (size_t)len);
        if (m.key.find('\0') != std::string::npos) return refuse(f, "a metadata key holds a zero byte");
        for (uint64_t j = 0; j < i; ++j)
            if (f->meta[(size_t)j].key == m.key) return refuse(f, "a metadata key appears twice");
        if (value(f, &m) != 0) return 2;
        if (m.key == "general.alignment") {
            if (m.type != AOTX_GGUF_U32) return refuse(f, "general.alignment is not a u32");
            if (m.u == 0 || (m.u & (m.u - 1u)) != 0 || m.u > 65536u)
                return refuse(f, "general.alignment is not a power of two");
            f->alignment = (uint32_t)m.u;
            have_align = true;
        }
    }
    (void)have_align;
    f->tensors.resize((size_t)tensors);
    f->streams.assign((size_t)tensors, false);
    for (uint64_t i = 0; i < tensors; ++i) {
        aotx_tensor_info &t = f->tensors[(size_t)i];
        memset(&t, 0, sizeof t);
        uint64_t at = 0, len = 0, dims = 0, type = 0, off = 0;
        if (string_at(f, &at, &len) != 0) return 2;
        if (len == 0 || len >= AOTX_TENSOR_NAME_BYTES) return refuse(f, "a tensor name is empty or too long");
        memcpy(t.name, f->head.data() + at, (size_t)len);
        t.name[len] = '\0';
        if (strlen(t.name) != len) return refuse(f, "a tensor name holds a zero byte");
        if (number(f, 4, &dims) != 0) return 2;
        if (dims == 0 || dims > AOTX_TENSOR_DIMS) return refuse(f, "a tensor has no dimensions or more than 4");
        t.dim_count = (uint32_t)dims;
        uint64_t weights = 1;
        for (uint32_t d = 0; d < AOTX_TENSOR_DIMS; ++d) t.dims[d] = 1;
        for (uint32_t d = 0; d < t.dim_count; ++d) {
            if (number(f, 8, &t.dims[d]) != 0) return 2;
            if (t.dims[d] == 0) return refuse(f, "a tensor dimension is zero");
            if (weights > UINT64_MAX / t.dims[d]) return refuse(f, "a tensor size overflows");
            weights *= t.dims[d];
        }
        if (number(f, 4, &type) != 0 || number(f, 8, &off) != 0) return 2;
        t.type = (uint32_t)type;
        t.offset = off;
        uint64_t bw = 0, bb = 0;
        if (tensor_block(t.type, &bw, &bb)) {
            if (t.dims[0] % bw != 0) return refuse(f, "a tensor row is not a whole number of blocks");
            if (weights / bw > UINT64_MAX / bb) return refuse(f, "a tensor size overflows");
            t.bytes = weights / bw * bb;
            f->streams[(size_t)i] = true;
        }
        for (uint64_t j = 0; j < i; ++j)
            if (strcmp(f->tensors[(size_t)j].name, t.name) == 0) return refuse(f, "a tensor name appears twice");
    }
    /* the tensor bytes start at the next multiple of the alignment */
    const uint64_t a = f->alignment;
    if (f->pos > UINT64_MAX - a) return refuse(f, "the head overflows");
    f->data_offset = (f->pos + a - 1u) / a * a;
    if (f->data_offset > f->file_bytes) return refuse(f, "the file ends before its tensor bytes");
    f->data_bytes = f->file_bytes - f->data_offset;
    for (const aotx_tensor_info &t : f->tensors) {
        if (t.offset % a != 0) return refuse(f, "a tensor offset is off the alignment");
        if (t.offset > f->data_bytes || t.bytes > f->data_bytes - t.offset)
            return refuse(f, "a tensor runs past the end of the file");
    }
    return 0;
}

const Meta *find_meta(const aotx_modelfile *f, const char *key)
{
    if (f == nullptr || key == nullptr) return nullptr;
    for (const Meta &m : f->meta)
        if (m.key == key) return &m;
    return nullptr;
}

bool is_unsigned(uint32_t t)
{
    return t == AOTX_GGUF_U8 || t == AOTX_GGUF_U16 || t == AOTX_GGUF_U32 || t == AOTX_GGUF_U64
        || t == AOTX_GGUF_BOOL;
}

bool is_signed(uint32_t t)
{
    return t == AOTX_GGUF_I8 || t == AOTX_GGUF_I16 || t == AOTX_GGUF_I32 || t == AOTX_GGUF_I64;
}

} // namespace

extern "C" int aotx_modelfile_open(const char *path, aotx_modelfile **file)
{
    if (file == nullptr) return 1;
    *file = nullptr;
    if (path == nullptr) return 1;
    aotx_modelfile *f = new (std::nothrow) aotx_modelfile();
    if (f == nullptr) return 1;
    f->path = path;
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (f->fd < 0 || fstat(f->fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        if (f->fd >= 0) close(f->fd);
        delete f;
        return 1;
    }
    f->file_bytes = (uint64_t)st.st_size;
    int rc = parse(f);
    std::vector<uint8_t>().swap(f->head);   /* the head is not kept */
    if (rc != 0) {
        close(f->fd);
        delete f;
        return rc;
    }
    *file = f;
    return 0;
}

extern "C" void aotx_modelfile_close(aotx_modelfile *file)
{
    if (file == nullptr) return;
    if (file->fd >= 0) close(file->fd);
    delete file;
}

extern "C" uint64_t aotx_modelfile_file_bytes(const aotx_modelfile *file)
{
    return file != nullptr ? file->file_bytes : 0u;
}

extern "C" uint64_t aotx_modelfile_header_bytes(const aotx_modelfile *file)
{
    return file != nullptr ? file->data_offset : 0u;
}

extern "C" int aotx_modelfile_u32(const aotx_modelfile *file, const char *key, uint32_t *value)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (value == nullptr) return 2;
    if (is_unsigned(m->type) || (is_signed(m->type) && !m->negative)) {
        if (m->u > UINT32_MAX) return 2;
        *value = (uint32_t)m->u;
        return 0;
    }
    return 2;
}

extern "C" int aotx_modelfile_u64(const aotx_modelfile *file, const char *key, uint64_t *value)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (value == nullptr) return 2;
    if (is_unsigned(m->type) || (is_signed(m->type) && !m->negative)) {
        *value = m->u;
        return 0;
    }
    return 2;
}

extern "C" int aotx_modelfile_f32(const aotx_modelfile *file, const char *key, float *value)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (value == nullptr || (m->type != AOTX_GGUF_F32 && m->type != AOTX_GGUF_F64)) return 2;
    *value = (float)m->f;
    return 0;
}

extern "C" int aotx_modelfile_string(const aotx_modelfile *file, const char *key,
                                     const char **value, size_t *length)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (value == nullptr || length == nullptr || m->type != AOTX_GGUF_STRING) return 2;
    *value = m->text.c_str();
    *length = m->text.size();
    return 0;
}

extern "C" int aotx_modelfile_strings(const aotx_modelfile *file, const char *key,
                                      aotx_string_array *array)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (array == nullptr || m->type != AOTX_GGUF_ARRAY || m->element_type != AOTX_GGUF_STRING)
        return 2;
    array->count = m->count;
    array->bytes = m->run.data();
    array->offsets = m->offsets.data();
    return 0;
}

extern "C" int aotx_modelfile_i32s(const aotx_modelfile *file, const char *key,
                                   const int32_t **values, uint64_t *count)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (values == nullptr || count == nullptr || m->type != AOTX_GGUF_ARRAY
        || m->element_type != AOTX_GGUF_I32)
        return 2;
    *values = m->i32.data();
    *count = m->count;
    return 0;
}

extern "C" int aotx_modelfile_f32s(const aotx_modelfile *file, const char *key,
                                   const float **values, uint64_t *count)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (values == nullptr || count == nullptr || m->type != AOTX_GGUF_ARRAY
        || m->element_type != AOTX_GGUF_F32)
        return 2;
    *values = m->f32.data();
    *count = m->count;
    return 0;
}

extern "C" int aotx_modelfile_bools(const aotx_modelfile *file, const char *key,
                                    const uint8_t **values, uint64_t *count)
{
    const Meta *m = find_meta(file, key);
    if (m == nullptr) return 1;
    if (values == nullptr || count == nullptr || m->type != AOTX_GGUF_ARRAY
        || m->element_type != AOTX_GGUF_BOOL)
        return 2;
    *values = m->run.data();
    *count = m->count;
    return 0;
}

extern "C" uint64_t aotx_modelfile_tensor_count(const aotx_modelfile *file)
{
    return file != nullptr ? (uint64_t)file->tensors.size() : 0u;
}

extern "C" int aotx_modelfile_tensor(const aotx_modelfile *file, uint64_t index,
                                     aotx_tensor_info *info)
{
    if (file == nullptr || info == nullptr) return 2;
    if (index >= file->tensors.size()) return 1;
    *info = file->tensors[(size_t)index];
    return 0;
}

extern "C" int aotx_modelfile_find(const aotx_modelfile *file, const char *name,
                                   aotx_tensor_info *info)
{
    if (file == nullptr || name == nullptr || info == nullptr) return 2;
    for (const aotx_tensor_info &t : file->tensors) {
        if (strcmp(t.name, name) == 0) {
            *info = t;
            return 0;
        }
    }
    return 1;
}

extern "C" uint64_t aotx_modelfile_data_bytes(const aotx_modelfile *file)
{
    return file != nullptr ? file->data_bytes : 0u;
}

extern "C" int aotx_modelfile_read(const aotx_modelfile *file, uint64_t offset, uint64_t bytes,
                                   void *buffer)
{
    if (file == nullptr || (buffer == nullptr && bytes != 0u)) return 2;
    if (offset > file->data_bytes || bytes > file->data_bytes - offset) return 2;
    uint8_t *out = (uint8_t *)buffer;
    uint64_t done = 0;
    while (done < bytes) {
        size_t want = (size_t)((bytes - done) < (1ull << 30) ? (bytes - done) : (1ull << 30));
        ssize_t got = pread(file->fd, out + done, want, (off_t)(file->data_offset + offset + done));
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return 1;
        done += (uint64_t)got;
    }
    return 0;
}

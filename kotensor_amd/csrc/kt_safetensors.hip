// kt_safetensors.hip -- reading and writing the reference's saveQuantized files
// (safetensors) for device-resident quantized weights. Host code only: the file is
// mapped read-only and tensor bytes go straight from the mapping into the caller's
// device buffers, in the layout the kernels consume (no repacking).
//
// Reader: SafeTensorsFile (Engine/kotensor/src/main/kotlin/SafeTensors.kt:12-107) and
// QuantizedTensor.mapFrom (QuantizedTensor.kt:109-125), with their checks and messages.
// Writer: SafeTensors.saveEntries (SafeTensors.kt:204-249): the same header text (key
// order, number formatting, string escapes), space padding to 8 bytes and data order,
// so that files re-save byte for byte.
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <utility>
#include <vector>

#include "kt_common.h"

namespace kt {
namespace {

// ---- a JSON reader for the header (objects, arrays, strings, numbers, literals) ------

struct JValue {
    enum Kind { OBJECT, ARRAY, STRING, NUMBER, LITERAL } kind = LITERAL;
    std::string text;  // STRING: decoded; NUMBER / LITERAL: as written
    std::vector<std::pair<std::string, JValue>> members;
    std::vector<JValue> items;
};

struct JParser {
    const char* p;
    const char* end;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t* v) {
        if (end - p < 4) return false;
        uint32_t r = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = p[i];
            r <<= 4;
            if (c >= '0' && c <= '9') r |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') r |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') r |= static_cast<uint32_t>(c - 'A' + 10);
            else return false;
        }
        p += 4;
        *v = r;
        return true;
    }
    bool string(std::string& out) {
        if (p >= end || *p != '"') return false;
        ++p;
        while (p < end && *p != '"') {
            if (*p != '\\') {
                out += *p++;
                continue;
            }
            if (++p >= end) return false;
            const char e = *p++;
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
                    uint32_t cp = 0;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        uint32_t lo = 0;
                        if (!hex4(&lo)) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: return false;
            }
        }
        if (p >= end) return false;
        ++p;
        return true;
    }
    bool value(JValue& v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p >= end) return false;
        if (*p == '{') {
            v.kind = JValue::OBJECT;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return true;
            }
            while (true) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p >= end || *p != ':') return false;
                ++p;
                JValue member;
                if (!value(member, depth + 1)) return false;
                v.members.emplace_back(std::move(key), std::move(member));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return true;
                }
                return false;
            }
        }
        if (*p == '[') {
            v.kind = JValue::ARRAY;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            while (true) {
                JValue item;
                if (!value(item, depth + 1)) return false;
                v.items.push_back(std::move(item));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return true;
                }
                return false;
            }
        }
        if (*p == '"') {
            v.kind = JValue::STRING;
            return string(v.text);
        }
        const char* start = p;
        if (*p == '-' || (*p >= '0' && *p <= '9')) {
            v.kind = JValue::NUMBER;
            while (p < end && (*p == '-' || *p == '+' || *p == '.' || *p == 'e' || *p == 'E' || (*p >= '0' && *p <= '9')))
                ++p;
        } else {
            v.kind = JValue::LITERAL;
            while (p < end && *p >= 'a' && *p <= 'z') ++p;
            const std::string lit(start, p);
            if (lit != "true" && lit != "false" && lit != "null") return false;
        }
        v.text.assign(start, p);
        return p > start;
    }
};

// An integer JSON number (shapes and offsets); false for fractions or overflow.
bool as_int64(const JValue& v, int64_t* out) {
    if (v.kind != JValue::NUMBER || v.text.empty()) return false;
    const char* s = v.text.c_str();
    bool neg = *s == '-';
    if (neg) ++s;
    if (!*s) return false;
    int64_t r = 0;
    for (; *s; ++s) {
        if (*s < '0' || *s > '9') return false;
        if (r > (INT64_MAX - (*s - '0')) / 10) return false;
        r = r * 10 + (*s - '0');
    }
    *out = neg ? -r : r;
    return true;
}

const JValue* member(const JValue& obj, const char* key) {
    for (const auto& m : obj.members)
        if (m.first == key) return &m.second;
    return nullptr;
}

// JSON text of a string, as the reference writes it (SafeTensors.kt:251-265): quote,
// backslash, \n, \r, \t escaped; other characters below 0x20 as \u00XX.
std::string json_string(const char* text) {
    std::string out = "\"";
    for (const unsigned char* c = reinterpret_cast<const unsigned char*>(text); *c; ++c) {
        switch (*c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (*c < 0x20) {
                    char buf[8];
                    snprintf(buf, sizeof buf, "\\u%04x", *c);
                    out += buf;
                } else {
                    out += static_cast<char>(*c);
                }
        }
    }
    return out + "\"";
}

int32_t copy_text(const std::string& s, char* buf, size_t len) {
    if (!buf || len == 0) return fail(KT_ERR_ARGUMENT, "output buffer is NULL or empty");
    if (s.size() + 1 > len) return fail(KT_ERR_ARGUMENT, "output buffer of %zu bytes is too small for %zu", len, s.size() + 1);
    memcpy(buf, s.c_str(), s.size() + 1);
    return KT_OK;
}

struct Entry {
    std::string name, dtype;
    std::vector<int64_t> shape;
    int64_t start = 0, end = 0;  // data_offsets
};

}  // namespace
}  // namespace kt

struct kt_st_file {
    std::string path;
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    int64_t data_start = 0;
    std::vector<kt::Entry> entries;
    std::vector<std::pair<std::string, std::string>> metadata;

    const kt::Entry* find(const char* name) const {
        for (const auto& e : entries)
            if (e.name == name) return &e;
        return nullptr;
    }
};

struct kt_st_writer {
    struct Item {
        std::string name, dtype;
        std::vector<int64_t> shape;
        const void* data;
        int64_t nbytes;
        bool on_device;
    };
    std::vector<std::pair<std::string, std::string>> metadata;
    std::vector<Item> items;
};

namespace {

void close_file(kt_st_file* f) {
    if (f->map) munmap(const_cast<uint8_t*>(f->map), f->size);
    if (f->fd >= 0) ::close(f->fd);
    delete f;
}

int32_t entry_or_fail(const kt_st_file* f, const std::string& name, const kt::Entry** e) {
    *e = f->find(name.c_str());
    if (!*e) return kt::fail(KT_ERR_ARGUMENT, "No tensor named '%s' in %s", name.c_str(), f->path.c_str());
    return KT_OK;
}

}  // namespace

using kt::fail;

extern "C" {

int32_t kt_st_open(const char* path, kt_st_file** file) {
    if (!path || !file) return fail(KT_ERR_ARGUMENT, "path or file is NULL");
    *file = nullptr;
    kt_st_file* f = new kt_st_file();
    f->path = path;
    f->fd = ::open(path, O_RDONLY);
    if (f->fd < 0) {
        delete f;
        return fail(KT_ERR_ARGUMENT, "%s (No such file or directory)", path);
    }
    struct stat st;
    if (fstat(f->fd, &st) != 0 || st.st_size < 8) {
        const long long sz = static_cast<long long>(st.st_size);
        close_file(f);
        return fail(KT_ERR_ARGUMENT, "%s holds %lld bytes, fewer than a safetensors header size", path, sz);
    }
    f->size = static_cast<size_t>(st.st_size);
    void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) {
        f->map = nullptr;
        close_file(f);
        return fail(KT_ERR_ARGUMENT, "cannot map %s", path);
    }
    f->map = static_cast<const uint8_t*>(m);
    int64_t header_size = 0;
    memcpy(&header_size, f->map, 8);  // little-endian, as the host
    if (header_size < 1 || header_size > (int64_t{100} << 20)) {
        close_file(f);
        return fail(KT_ERR_ARGUMENT, "Invalid safetensors header size %lld in %s", static_cast<long long>(header_size), path);
    }
    if (8 + header_size > static_cast<int64_t>(f->size)) {
        close_file(f);
        return fail(KT_ERR_ARGUMENT, "safetensors header of %s runs past the end of the file", path);
    }
    f->data_start = 8 + header_size;
    kt::JParser parser{reinterpret_cast<const char*>(f->map) + 8, reinterpret_cast<const char*>(f->map) + 8 + header_size};
    kt::JValue root;
    const bool parsed = parser.value(root, 0);
    if (parsed) parser.ws();
    if (!parsed || root.kind != kt::JValue::OBJECT) {
        close_file(f);
        return fail(KT_ERR_ARGUMENT, "safetensors header of %s is not a JSON object", path);
    }
    for (const auto& m : root.members) {
        const std::string& name = m.first;
        const kt::JValue& body = m.second;
        if (body.kind != kt::JValue::OBJECT) continue;
        if (name == "__metadata__") {
            for (const auto& kv : body.members) f->metadata.emplace_back(kv.first, kv.second.text);
            continue;
        }
        kt::Entry e;
        e.name = name;
        const kt::JValue* dtype = kt::member(body, "dtype");
        if (!dtype || dtype->kind != kt::JValue::STRING) {
            close_file(f);
            return fail(KT_ERR_ARGUMENT, "Tensor %s has no dtype", name.c_str());
        }
        e.dtype = dtype->text;
        if (const kt::JValue* shape = kt::member(body, "shape")) {
            for (const auto& d : shape->items) {
                int64_t v = 0;
                if (!kt::as_int64(d, &v)) {
                    close_file(f);
                    return fail(KT_ERR_ARGUMENT, "Tensor %s has a shape that is not a list of integers", name.c_str());
                }
                e.shape.push_back(v);
            }
        }
        const kt::JValue* offsets = kt::member(body, "data_offsets");
        if (!offsets || offsets->kind != kt::JValue::ARRAY || offsets->items.size() < 2 ||
            !kt::as_int64(offsets->items[0], &e.start) || !kt::as_int64(offsets->items[1], &e.end)) {
            close_file(f);
            return fail(KT_ERR_ARGUMENT, "Tensor %s has no data_offsets", name.c_str());
        }
        // data_start <= size holds (checked above), so the right side cannot overflow; an
        // end near INT64_MAX must not wrap into a small sum.
        if (!(e.end >= e.start && e.start >= 0 && e.end <= static_cast<int64_t>(f->size) - f->data_start)) {
            const long long s = e.start, en = e.end, sz = static_cast<long long>(f->size);
            close_file(f);
            return fail(KT_ERR_ARGUMENT, "Tensor %s data range [%lld, %lld) exceeds file %lld", name.c_str(), s, en, sz);
        }
        f->entries.push_back(std::move(e));
    }
    *file = f;
    return KT_OK;
}

int32_t kt_st_close(kt_st_file* file) {
    if (file) close_file(file);
    return KT_OK;
}

int32_t kt_st_count(const kt_st_file* file, int32_t* count) {
    if (!file || !count) return fail(KT_ERR_ARGUMENT, "file or count is NULL");
    *count = static_cast<int32_t>(file->entries.size());
    return KT_OK;
}

int32_t kt_st_name(const kt_st_file* file, int32_t index, char* buf, size_t len) {
    if (!file) return fail(KT_ERR_ARGUMENT, "file is NULL");
    if (index < 0 || index >= static_cast<int32_t>(file->entries.size()))
        return fail(KT_ERR_RANGE, "entry index %d out of range [0, %zu)", index, file->entries.size());
    return kt::copy_text(file->entries[index].name, buf, len);
}

int32_t kt_st_find(const kt_st_file* file, const char* name, kt_st_entry* entry) {
    if (!file || !name || !entry) return fail(KT_ERR_ARGUMENT, "file, name or entry is NULL");
    const kt::Entry* e = nullptr;
    if (int32_t st = entry_or_fail(file, name, &e)) return st;
    if (e->dtype.size() >= sizeof entry->dtype) return fail(KT_ERR_ARGUMENT, "Tensor %s has dtype '%s'", name, e->dtype.c_str());
    if (e->shape.size() > 8) return fail(KT_ERR_ARGUMENT, "Tensor %s has %zu dimensions, more than 8", name, e->shape.size());
    memset(entry, 0, sizeof *entry);
    memcpy(entry->dtype, e->dtype.c_str(), e->dtype.size() + 1);
    entry->rank = static_cast<int32_t>(e->shape.size());
    for (size_t i = 0; i < e->shape.size(); ++i) entry->shape[i] = e->shape[i];
    entry->offset = file->data_start + e->start;
    entry->nbytes = e->end - e->start;
    return KT_OK;
}

int32_t kt_st_metadata(const kt_st_file* file, const char* key, char* buf, size_t len) {
    if (!file || !key) return fail(KT_ERR_ARGUMENT, "file or key is NULL");
    for (const auto& kv : file->metadata)
        if (kv.first == key) return kt::copy_text(kv.second, buf, len);
    return fail(KT_ERR_ARGUMENT, "%s has no %s metadata", file->path.c_str(), key);
}

int32_t kt_st_metadata_key(const kt_st_file* file, int32_t index, char* buf, size_t len) {
    if (!file) return fail(KT_ERR_ARGUMENT, "file is NULL");
    if (index < 0 || index >= static_cast<int32_t>(file->metadata.size()))
        return fail(KT_ERR_RANGE, "metadata index %d out of range [0, %zu)", index, file->metadata.size());
    return kt::copy_text(file->metadata[index].first, buf, len);
}

int32_t kt_st_data(const kt_st_file* file, const char* name, const void** data, int64_t* nbytes) {
    if (!file || !name || !data || !nbytes) return fail(KT_ERR_ARGUMENT, "file, name, data or nbytes is NULL");
    const kt::Entry* e = nullptr;
    if (int32_t st = entry_or_fail(file, name, &e)) return st;
    *data = file->map + file->data_start + e->start;
    *nbytes = e->end - e->start;
    return KT_OK;
}

int32_t kt_st_load_qweight(const kt_st_file* file, const char* name, const kt_qweight* w, void* stream) {
    if (!file || !name || !w) return fail(KT_ERR_ARGUMENT, "file, name or weight is NULL");
    kt::WeightView v;
    if (int32_t st = kt::view_weight(w, &v)) return st;
    const std::string base = name;
    const kt::Entry *q = nullptr, *s = nullptr, *z = nullptr;
    if (int32_t st = entry_or_fail(file, base + ".qweight", &q)) return st;
    const long long q_expected = static_cast<long long>(v.K) * v.bpr;
    if (q->end - q->start != q_expected)
        return fail(KT_ERR_SHAPE, "%s.qweight has %lld bytes, expected %lld", name, static_cast<long long>(q->end - q->start),
                    q_expected);
    if (int32_t st = entry_or_fail(file, base + ".scales", &s)) return st;
    const long long s_expected = static_cast<long long>(v.G) * v.N * 4;
    if (s->dtype != "F32" || s->end - s->start != s_expected)
        return fail(KT_ERR_SHAPE, "%s.scales is %s with %lld bytes, expected F32 with %lld", name, s->dtype.c_str(),
                    static_cast<long long>(s->end - s->start), s_expected);
    if (w->zeros) {
        if (int32_t st = entry_or_fail(file, base + ".zeros", &z)) return st;
        const long long z_expected = static_cast<long long>(v.G) * v.N;
        if (z->end - z->start != z_expected)
            return fail(KT_ERR_SHAPE, "%s.zeros has %lld bytes, expected %lld", name, static_cast<long long>(z->end - z->start),
                        z_expected);
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint8_t* data = file->map + file->data_start;
    KT_HIP(hipMemcpyAsync(const_cast<void*>(w->qdata), data + q->start, q->end - q->start, hipMemcpyHostToDevice, st));
    KT_HIP(hipMemcpyAsync(const_cast<float*>(w->scales), data + s->start, s->end - s->start, hipMemcpyHostToDevice, st));
    if (z) KT_HIP(hipMemcpyAsync(const_cast<uint8_t*>(w->zeros), data + z->start, z->end - z->start, hipMemcpyHostToDevice, st));
    KT_HIP(hipStreamSynchronize(st));
    return KT_OK;
}

int32_t kt_st_writer_create(kt_st_writer** writer) {
    if (!writer) return fail(KT_ERR_ARGUMENT, "writer is NULL");
    *writer = new kt_st_writer();
    return KT_OK;
}

int32_t kt_st_writer_destroy(kt_st_writer* writer) {
    delete writer;
    return KT_OK;
}

int32_t kt_st_writer_metadata(kt_st_writer* writer, const char* key, const char* value) {
    if (!writer || !key || !value) return fail(KT_ERR_ARGUMENT, "writer, key or value is NULL");
    for (auto& kv : writer->metadata)
        if (kv.first == key) {  // a map: a repeated key keeps its first position
            kv.second = value;
            return KT_OK;
        }
    writer->metadata.emplace_back(key, value);
    return KT_OK;
}

int32_t kt_st_writer_add(kt_st_writer* writer, const char* name, const char* dtype, int32_t rank, const int64_t* shape,
                         const void* data, int64_t nbytes, int32_t on_device) {
    if (!writer || !name || !dtype) return fail(KT_ERR_ARGUMENT, "writer, name or dtype is NULL");
    if (rank < 0 || rank > 8 || (rank > 0 && !shape)) return fail(KT_ERR_ARGUMENT, "rank %d needs 0..8 dimensions", rank);
    if (nbytes < 0 || (nbytes > 0 && !data)) return fail(KT_ERR_ARGUMENT, "entry %s has %lld bytes at NULL", name,
                                                          static_cast<long long>(nbytes));
    kt_st_writer::Item it;
    it.name = name;
    it.dtype = dtype;
    it.shape.assign(shape, shape + rank);
    it.data = data;
    it.nbytes = nbytes;
    it.on_device = on_device != 0;
    writer->items.push_back(std::move(it));
    return KT_OK;
}

int32_t kt_st_writer_add_qweight(kt_st_writer* writer, const char* name, const kt_qweight* w) {
    if (!writer || !name || !w) return fail(KT_ERR_ARGUMENT, "writer, name or weight is NULL");
    kt::WeightView v;
    if (int32_t st = kt::view_weight(w, &v)) return st;
    const std::string base = name;
    const int64_t qshape[2] = {v.K, v.bpr};
    const int64_t gshape[2] = {v.G, v.N};
    if (int32_t st = kt_st_writer_add(writer, (base + ".qweight").c_str(), v.bits == 8 ? "I8" : "U8", 2, qshape, w->qdata,
                                      static_cast<int64_t>(v.K) * v.bpr, 1))
        return st;
    if (int32_t st = kt_st_writer_add(writer, (base + ".scales").c_str(), "F32", 2, gshape, w->scales,
                                      static_cast<int64_t>(v.G) * v.N * 4, 1))
        return st;
    if (w->zeros)
        return kt_st_writer_add(writer, (base + ".zeros").c_str(), "U8", 2, gshape, w->zeros, static_cast<int64_t>(v.G) * v.N, 1);
    return KT_OK;
}

int32_t kt_st_writer_save(kt_st_writer* writer, const char* path, void* stream) {
    if (!writer || !path) return fail(KT_ERR_ARGUMENT, "writer or path is NULL");
    // Header text of SafeTensors.saveEntries (SafeTensors.kt:208-224).
    std::vector<std::string> parts;
    if (!writer->metadata.empty()) {
        std::string pairs;
        for (size_t i = 0; i < writer->metadata.size(); ++i) {
            if (i) pairs += ",";
            pairs += kt::json_string(writer->metadata[i].first.c_str()) + ":" + kt::json_string(writer->metadata[i].second.c_str());
        }
        parts.push_back("\"__metadata__\":{" + pairs + "}");
    }
    long long offset = 0;
    for (const auto& it : writer->items) {
        std::string shape;
        for (size_t i = 0; i < it.shape.size(); ++i) {
            if (i) shape += ",";
            shape += std::to_string(it.shape[i]);
        }
        const long long start = offset, end = offset + it.nbytes;
        parts.push_back(kt::json_string(it.name.c_str()) + ":{\"dtype\":\"" + it.dtype + "\",\"shape\":[" + shape +
                        "],\"data_offsets\":[" + std::to_string(start) + "," + std::to_string(end) + "]}");
        offset = end;
    }
    std::string header = "{";
    for (size_t i = 0; i < parts.size(); ++i) {
        if (i) header += ",";
        header += parts[i];
    }
    header += "}";
    const size_t padding = (8 - header.size() % 8) % 8;
    const int64_t header_size = static_cast<int64_t>(header.size() + padding);

    FILE* out = fopen(path, "wb");
    if (!out) return fail(KT_ERR_ARGUMENT, "cannot write %s", path);
    bool ok = fwrite(&header_size, 8, 1, out) == 1 && fwrite(header.data(), 1, header.size(), out) == header.size();
    for (size_t i = 0; ok && i < padding; ++i) ok = fputc(' ', out) != EOF;
    hipStream_t st = static_cast<hipStream_t>(stream);
    std::vector<uint8_t> staging;
    for (const auto& it : writer->items) {
        if (!ok) break;
        const void* src = it.data;
        if (it.on_device && it.nbytes > 0) {
            staging.resize(static_cast<size_t>(it.nbytes));
            hipError_t e = hipMemcpyAsync(staging.data(), it.data, static_cast<size_t>(it.nbytes), hipMemcpyDeviceToHost, st);
            if (e == hipSuccess) e = hipStreamSynchronize(st);
            if (e != hipSuccess) {
                fclose(out);
                return kt::hip_fail(e, "kt_st_writer_save: device read");
            }
            src = staging.data();
        }
        if (it.nbytes > 0) ok = fwrite(src, 1, static_cast<size_t>(it.nbytes), out) == static_cast<size_t>(it.nbytes);
    }
    if (fclose(out) != 0) ok = false;
    if (!ok) return fail(KT_ERR_ARGUMENT, "cannot write %s", path);
    return KT_OK;
}

}  // extern "C"

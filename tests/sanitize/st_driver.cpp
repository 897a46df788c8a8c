// Host sanitizer driver for the safetensors reader and writer of libkotensor_hip.so (test
// infrastructure): writes a file from host tensors, reads it back, then opens malformed
// files (truncated, header past the end, offsets out of range or overflowing, bad JSON,
// duplicate names, a rank above 8) that must fail with a status, never a crash, under
// AddressSanitizer + UndefinedBehaviorSanitizer (see run.sh). No GPU is used.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/kotensor_hip.h"

static int failures = 0;
#define EXPECT(c)                                                        \
    do {                                                                 \
        if (!(c)) {                                                      \
            fprintf(stderr, "st driver: line %d: %s\n", __LINE__, #c);   \
            ++failures;                                                  \
        }                                                                \
    } while (0)

static void write_file(const std::string& path, const std::string& header, size_t data_bytes) {
    FILE* f = fopen(path.c_str(), "wb");
    uint64_t n = header.size();
    fwrite(&n, 8, 1, f);
    fwrite(header.data(), 1, header.size(), f);
    std::vector<char> zeros(data_bytes, 0);
    fwrite(zeros.data(), 1, zeros.size(), f);
    fclose(f);
}

static int open_status(const std::string& path) {
    kt_st_file* f = nullptr;
    const int32_t st = kt_st_open(path.c_str(), &f);
    if (st == KT_OK) {
        int32_t count = 0;
        kt_st_count(f, &count);
        for (int32_t i = 0; i < count; ++i) {
            char name[256];
            kt_st_name(f, i, name, sizeof name);
            kt_st_entry e;
            kt_st_find(f, name, &e);
            const void* data = nullptr;
            int64_t nbytes = 0;
            kt_st_data(f, name, &data, &nbytes);
        }
        kt_st_close(f);
    }
    return st;
}

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    // a valid file from the writer
    const std::string good = dir + "/st_good.safetensors";
    {
        kt_st_writer* w = nullptr;
        EXPECT(kt_st_writer_create(&w) == KT_OK);
        EXPECT(kt_st_writer_metadata(w, "kotensor.quantization", "int4/g64") == KT_OK);
        EXPECT(kt_st_writer_metadata(w, "note", "quote \" backslash \\ tab \t end") == KT_OK);
        std::vector<float> a(6 * 5);
        for (size_t i = 0; i < a.size(); ++i) a[i] = 0.5f * static_cast<float>(i);
        std::vector<uint8_t> b(7);
        const int64_t sa[2] = {6, 5}, sb[1] = {7};
        EXPECT(kt_st_writer_add(w, "layers.0.w", "F32", 2, sa, a.data(), 4 * 30, 0) == KT_OK);
        EXPECT(kt_st_writer_add(w, "bytes", "U8", 1, sb, b.data(), 7, 0) == KT_OK);
        EXPECT(kt_st_writer_save(w, good.c_str(), nullptr) == KT_OK);
        kt_st_writer_destroy(w);
        // the writer, like SafeTensors.saveEntries, writes what it is given: a repeated name
        // and a byte count that disagrees with the shape go into the file, and reading
        // that file back must end in a status either way
        EXPECT(kt_st_writer_create(&w) == KT_OK);
        EXPECT(kt_st_writer_add(w, "bytes", "U8", 1, sb, b.data(), 7, 0) == KT_OK);
        EXPECT(kt_st_writer_add(w, "bytes", "U8", 1, sb, b.data(), 7, 0) == KT_OK);
        EXPECT(kt_st_writer_add(w, "odd", "F32", 2, sa, a.data(), 4, 0) == KT_OK);
        const std::string odd = dir + "/st_odd.safetensors";
        EXPECT(kt_st_writer_save(w, odd.c_str(), nullptr) == KT_OK);
        kt_st_writer_destroy(w);
        printf("st driver: duplicate / mismatched entries read back with status %d\n", open_status(odd));
    }
    EXPECT(open_status(good) == KT_OK);
    {
        kt_st_file* f = nullptr;
        EXPECT(kt_st_open(good.c_str(), &f) == KT_OK);
        char buf[8];  // a buffer too small is refused, never overrun
        EXPECT(kt_st_metadata(f, "note", buf, sizeof buf) != KT_OK);
        char big[256];
        EXPECT(kt_st_metadata(f, "note", big, sizeof big) == KT_OK);
        EXPECT(strcmp(big, "quote \" backslash \\ tab \t end") == 0);
        EXPECT(kt_st_name(f, 0, big, sizeof big) == KT_OK);
        kt_st_entry e;
        EXPECT(kt_st_find(f, "missing", &e) != KT_OK);
        EXPECT(kt_st_name(f, 99, buf, sizeof buf) != KT_OK);
        kt_st_close(f);
    }
    // malformed files: each must be refused with a status
    const std::string bad = dir + "/st_bad.safetensors";
    const std::vector<std::pair<std::string, size_t>> cases = {
        {"{", 0},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8]}", 8},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,9]}}", 8},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[8,0]}}", 8},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,18446744073709551615]}}", 8},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[-8,0]}}", 8},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[1,1,1,1,1,1,1,1,2],\"data_offsets\":[0,8]}}", 8},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8]},\"a\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8]}}", 8},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[3],\"data_offsets\":[0,8]}}", 8},
        {"{\"a\":{\"dtype\":\"F32XXXXXXXX\",\"shape\":[2],\"data_offsets\":[0,8]}}", 8},
        {"{\"__metadata__\":{\"k\":\"\\u00zz\"}}", 0},
        {"{\"a\":{\"dtype\":\"F32\",\"shape\":[99999999999999999999],\"data_offsets\":[0,8]}}", 8},
        {std::string(64, '['), 0},
    };
    // the first six break the format (truncated JSON, offsets outside the data, reversed,
    // overflowing or negative) and must be refused at open; the rest (a rank above 8,
    // repeated names, a shape that disagrees with its bytes, odd dtypes and escapes,
    // nesting) only have to end in a status: like SafeTensors.kt, open reads them and the
    // accessors or kt_st_load_qweight's size checks refuse what they cannot use
    for (size_t i = 0; i < cases.size(); ++i) {
        write_file(bad, cases[i].first, cases[i].second);
        const int32_t st = open_status(bad);
        printf("st driver: malformed case %zu -> status %d\n", i, st);
        if (i < 6) EXPECT(st != KT_OK);
    }
    // header length beyond the file, and a file shorter than the length field
    {
        FILE* f = fopen(bad.c_str(), "wb");
        const uint64_t n = 1u << 30;
        fwrite(&n, 8, 1, f);
        fwrite("{}", 1, 2, f);
        fclose(f);
        EXPECT(open_status(bad) != KT_OK);
        f = fopen(bad.c_str(), "wb");
        fwrite("abc", 1, 3, f);
        fclose(f);
        EXPECT(open_status(bad) != KT_OK);
    }
    EXPECT(open_status(dir + "/does_not_exist.safetensors") != KT_OK);
    printf("st driver: %s\n", failures ? "FAILED" : "ok");
    return failures != 0;
}

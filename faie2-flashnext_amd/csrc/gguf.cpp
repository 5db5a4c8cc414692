// GGUF reader: POSIX mmap of the file, then one pass over the header (gguf.h).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace fn {

void set_error(const std::string &msg);

namespace {

struct Cursor {
    const uint8_t *p, *end;
    bool ok = true;
    template <typename T> T get() {
        T v{};
        if (!ok || (size_t) (end - p) < sizeof(T)) {
            ok = false;
            return v;
        }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t) (end - p) < n) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p), n);
        p += n;
        return s;
    }
    void skip(uint64_t n) {
        if (!ok || (uint64_t) (end - p) < n) ok = false;
        else p += n;
    }
};

// GGUF value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64
size_t scalar_bytes(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

// a scalar as int64 (exact for every integer type) and as double
bool scalar(Cursor &c, uint32_t t, int64_t &i, double &d) {
    switch (t) {
        case 0: i = c.get<uint8_t>(); break;
        case 1: i = c.get<int8_t>(); break;
        case 2: i = c.get<uint16_t>(); break;
        case 3: i = c.get<int16_t>(); break;
        case 4: i = c.get<uint32_t>(); break;
        case 5: i = c.get<int32_t>(); break;
        case 7: i = c.get<uint8_t>() != 0; break;
        case 10: i = (int64_t) c.get<uint64_t>(); break;
        case 11: i = c.get<int64_t>(); break;
        case 6: d = c.get<float>(); i = (int64_t) d; return c.ok;
        case 12: d = c.get<double>(); i = (int64_t) d; return c.ok;
        default: return false;
    }
    d = (double) i;
    return c.ok;
}

}  // namespace

bool ggml_type_block(uint32_t type, int &values, int &bytes) {
    switch (type) {
        case 0: values = 1; bytes = 4; return true;      // F32
        case 1: values = 1; bytes = 2; return true;      // F16
        case 8: values = 32; bytes = 34; return true;    // Q8_0
        case 12: values = 256; bytes = 144; return true; // Q4_K
        case 13: values = 256; bytes = 176; return true; // Q5_K
        case 14: values = 256; bytes = 210; return true; // Q6_K
        case 16: values = 256; bytes = 66; return true;  // IQ2_XXS
        case 17: values = 256; bytes = 74; return true;  // IQ2_XS
        case 18: values = 256; bytes = 98; return true;  // IQ3_XXS
        case 20: values = 32; bytes = 18; return true;   // IQ4_NL
        case 21: values = 256; bytes = 110; return true; // IQ3_S
        case 22: values = 256; bytes = 82; return true;  // IQ2_S
        case 23: values = 256; bytes = 136; return true; // IQ4_XS
        case 30: values = 1; bytes = 2; return true;     // BF16
        case 42: values = 64; bytes = 18; return true;   // Q2_0 (the reference model's routed-expert down format)
        default: return false;
    }
}

Gguf::~Gguf() {
    if (base) munmap(const_cast<uint8_t *>(base), size);
}

int gguf_open(Gguf &g, const char *path) {
    if (!path || !*path) {
        set_error("gguf: no file name");
        return -1;
    }
    g.path = path;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_error(std::string("gguf: cannot open ") + path + ": " + std::strerror(errno));
        return -1;
    }
    struct stat st {};
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        set_error(std::string("gguf: ") + path + " is too short to be a GGUF file");
        return -1;
    }
    void *m = mmap(nullptr, (size_t) st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        set_error(std::string("gguf: mmap of ") + path + " failed: " + std::strerror(errno));
        return -1;
    }
    g.base = static_cast<const uint8_t *>(m);
    g.size = (uint64_t) st.st_size;

    Cursor c{g.base, g.base + g.size};
    if (c.get<uint32_t>() != 0x46554747u) {
        set_error(std::string("gguf: ") + path + " is not a GGUF file (bad magic)");
        return -1;
    }
    g.version = c.get<uint32_t>();
    if (g.version < 2 || g.version > 3) {
        set_error("gguf: version " + std::to_string(g.version) + " is not supported (2 or 3)");
        return -1;
    }
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (n_tensors > (1u << 24) || n_kv > (1u << 24)) {
        set_error("gguf: implausible tensor or key count");
        return -1;
    }
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        const std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (t == 8) {
            g.strs[key] = c.str();
        } else if (t == 9) {
            const uint32_t et = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (et == 8) {
                for (uint64_t j = 0; j < n && c.ok; ++j) c.str();
            } else if (const size_t eb = scalar_bytes(et)) {
                if (n > g.size) c.ok = false;
                auto &v = g.iarrays[key];
                for (uint64_t j = 0; j < n && c.ok; ++j) {
                    int64_t iv = 0;
                    double dv = 0;
                    if (!scalar(c, et, iv, dv)) c.ok = false;
                    v.push_back(iv);
                }
                (void) eb;
            } else {
                c.ok = false;
            }
        } else {
            int64_t iv = 0;
            double dv = 0;
            if (!scalar(c, t, iv, dv)) {
                c.ok = false;
                break;
            }
            g.nums[key] = dv;
            if (key == "general.alignment") g.alignment = (uint64_t) iv;
        }
    }
    if (!c.ok) {
        set_error("gguf: truncated or malformed key/value section in " + g.path);
        return -1;
    }
    if (g.alignment == 0 || (g.alignment & (g.alignment - 1))) {
        set_error("gguf: general.alignment must be a power of two");
        return -1;
    }
    std::vector<std::pair<std::string, GTensor>> infos;
    for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
        std::string name = c.str();
        GTensor t;
        const uint32_t nd = c.get<uint32_t>();
        if (nd < 1 || nd > 4) {
            c.ok = false;
            break;
        }
        t.nd = (int) nd;
        for (uint32_t d = 0; d < nd; ++d) t.ne[d] = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        infos.emplace_back(std::move(name), t);
    }
    if (!c.ok) {
        set_error("gguf: truncated or malformed tensor table in " + g.path);
        return -1;
    }
    const uint64_t pos = (uint64_t) (c.p - g.base);
    const uint64_t data0 = (pos + g.alignment - 1) / g.alignment * g.alignment;
    for (auto &kv : infos) {
        GTensor &t = kv.second;
        int qk = 0, bb = 0;
        if (!ggml_type_block(t.type, qk, bb)) {
            set_error("gguf: tensor " + kv.first + " has ggml type " + std::to_string(t.type) + ", not read here");
            return -1;
        }
        if (t.ne[0] % (uint64_t) qk) {
            set_error("gguf: tensor " + kv.first + ": rows are not whole blocks of its type");
            return -1;
        }
        // the byte count in 64 bits without wrapping (a header can claim any sizes)
        uint64_t rows = 0, row_bytes = 0;
        if (__builtin_mul_overflow(t.ne[1], t.ne[2], &rows) || __builtin_mul_overflow(rows, t.ne[3], &rows) ||
            __builtin_mul_overflow(t.ne[0] / (uint64_t) qk, (uint64_t) bb, &row_bytes) ||
            __builtin_mul_overflow(row_bytes, rows, &t.nbytes)) {
            set_error("gguf: tensor " + kv.first + " has implausible dimensions");
            return -1;
        }
        if (t.offset % g.alignment || data0 > g.size || t.offset > g.size - data0 ||
            t.nbytes > g.size - data0 - t.offset) {
            set_error("gguf: tensor " + kv.first + " lies outside the file or is misaligned");
            return -1;
        }
        t.data = g.base + data0 + t.offset;
        g.tensors[kv.first] = t;
    }
    return 0;
}

}  // namespace fn

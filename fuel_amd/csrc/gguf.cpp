// GGUF header parse over a read-only memory map (see gguf.hpp).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace frq {
namespace gguf {

File::~File() {
    if (map && map_bytes) munmap(const_cast<uint8_t*>(map), map_bytes);
}

// GgmlDType::from_u32 codes (fuel-ir/src/quantized.rs:36-58) and their
// block_size / type_size (:60-104).
size_t dtype_block_size(int t) {
    switch (t) {
        case 0: case 1: case 30: return 1;                                   // F32, F16, BF16
        case 2: case 3: case 6: case 7: case 8: case 9: return 32;          // Q4_0 .. Q8_1
        case 10: case 11: case 12: case 13: case 14: case 15: return 256;   // Q2K .. Q8K
        default: return 0;
    }
}

size_t dtype_type_size(int t) {
    switch (t) {
        case 0: return 4;
        case 1: case 30: return 2;
        case 2: return 18;
        case 3: return 20;
        case 6: return 22;
        case 7: return 24;
        case 8: return 34;
        case 9: return 36;
        case 10: return 84;
        case 11: return 110;
        case 12: return 144;
        case 13: return 176;
        case 14: return 210;
        case 15: return 292;
        default: return 0;
    }
}

namespace {

struct ParseError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void bail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void bail(const char* fmt, ...) {
    char buf[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw ParseError(buf);
}

// String::from_utf8_lossy: each maximal invalid subpart becomes U+FFFD.
std::string utf8_lossy(const uint8_t* p, size_t n) {
    std::string out;
    out.reserve(n);
    size_t i = 0;
    while (i < n) {
        const uint8_t b = p[i];
        if (b < 0x80) {
            out.push_back((char)b);
            i++;
            continue;
        }
        int len;
        uint8_t lo = 0x80, hi = 0xbf;  // range of the second byte
        if (b >= 0xc2 && b <= 0xdf) len = 2;
        else if (b == 0xe0) len = 3, lo = 0xa0;
        else if ((b >= 0xe1 && b <= 0xec) || b == 0xee || b == 0xef) len = 3;
        else if (b == 0xed) len = 3, hi = 0x9f;
        else if (b == 0xf0) len = 4, lo = 0x90;
        else if (b >= 0xf1 && b <= 0xf3) len = 4;
        else if (b == 0xf4) len = 4, hi = 0x8f;
        else len = 0;
        int k = 1;
        if (len) {
            for (; k < len; k++) {
                if (i + k >= n) break;
                const uint8_t c = p[i + k];
                const bool in = k == 1 ? (c >= lo && c <= hi) : (c >= 0x80 && c <= 0xbf);
                if (!in) break;
            }
        }
        if (len && k == len) {
            out.append(reinterpret_cast<const char*>(p + i), (size_t)len);
            i += (size_t)len;
        } else {
            out.append("\xef\xbf\xbd");
            i += (size_t)k;
        }
    }
    return out;
}

struct Reader {
    const uint8_t* p;
    size_t n;
    size_t pos = 0;
    int version = 0;

    void need(size_t k) {
        if (n - pos < k) bail("gguf: unexpected end of file at byte %zu (need %zu more)", pos, k);
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        memcpy(&v, p + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    // u32 counts / lengths in version 1, u64 from version 2
    uint64_t count() { return version == 1 ? (uint64_t)get<uint32_t>() : get<uint64_t>(); }

    std::string string() {
        const uint64_t len = count();
        need(len);
        size_t l = (size_t)len;
        const uint8_t* s = p + pos;
        pos += l;
        while (l && s[l - 1] == 0) l--;  // NUL terminators seen in practice are dropped
        return utf8_lossy(s, l);
    }

    Value value(uint32_t type) {
        Value v;
        v.type = (int)type;
        switch (type) {
            case VT_U8: v.u = get<uint8_t>(); break;
            case VT_I8: v.i = get<int8_t>(); break;
            case VT_U16: v.u = get<uint16_t>(); break;
            case VT_I16: v.i = get<int16_t>(); break;
            case VT_U32: v.u = get<uint32_t>(); break;
            case VT_I32: v.i = get<int32_t>(); break;
            case VT_U64: v.u = get<uint64_t>(); break;
            case VT_I64: v.i = get<int64_t>(); break;
            case VT_F32: v.f = (double)get<float>(); break;
            case VT_F64: v.f = get<double>(); break;
            case VT_BOOL: {
                const uint8_t b = get<uint8_t>();
                if (b > 1) bail("unexpected bool value %u", (unsigned)b);
                v.u = b;
                break;
            }
            case VT_STRING: v.s = string(); break;
            case VT_ARRAY: {
                const uint32_t et = value_type();
                const uint64_t len = count();
                if (len > n - pos) bail("gguf: array of %llu values exceeds the file", (unsigned long long)len);
                v.a.reserve((size_t)len);
                for (uint64_t j = 0; j < len; j++) v.a.push_back(value(et));
                break;
            }
            default: bail("unrecognized value-type %#08x", type);
        }
        return v;
    }

    uint32_t value_type() {
        const uint32_t t = get<uint32_t>();
        if (t > 12) bail("unrecognized value-type %#08x", t);
        return t;
    }
};

}  // namespace

std::unique_ptr<File> open(const char* path, std::string& err) {
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        err = std::string("gguf: cannot open ") + path + ": " + strerror(errno);
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        err = std::string("gguf: cannot stat ") + path + ": " + strerror(errno);
        ::close(fd);
        return nullptr;
    }
    std::unique_ptr<File> f(new File());
    f->map_bytes = (size_t)st.st_size;
    if (f->map_bytes) {
        void* m = mmap(nullptr, f->map_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            err = std::string("gguf: cannot map ") + path + ": " + strerror(errno);
            f->map_bytes = 0;
            ::close(fd);
            return nullptr;
        }
        f->map = static_cast<const uint8_t*>(m);
    }
    ::close(fd);  // the mapping stays valid

    try {
        Reader r{f->map, f->map_bytes};
        const uint32_t magic = r.get<uint32_t>();
        if (magic != 0x46554747u && magic != 0x47475546u) bail("unknown magic 0x%08x", magic);
        const uint32_t version = r.get<uint32_t>();
        if (version < 1 || version > 3) bail("gguf: unsupported magic/version Gguf/%u", version);
        r.version = f->version = (int)version;
        const uint64_t tensor_count = r.count();
        const uint64_t kv_count = r.count();
        for (uint64_t i = 0; i < kv_count; i++) {
            std::string key = r.string();
            const uint32_t t = r.value_type();
            Value v = r.value(t);
            auto it = f->meta_index.find(key);
            if (it != f->meta_index.end()) {
                f->metadata[it->second].second = std::move(v);
            } else {
                f->meta_index.emplace(key, f->metadata.size());
                f->metadata.emplace_back(std::move(key), std::move(v));
            }
        }
        for (uint64_t i = 0; i < tensor_count; i++) {
            TensorInfo ti;
            ti.name = r.string();
            const uint32_t nd = r.get<uint32_t>();
            r.need((size_t)nd * (version == 1 ? 4u : 8u));
            ti.dims.resize(nd);
            for (uint32_t d = 0; d < nd; d++) ti.dims[nd - 1 - d] = r.count();  // reversed: outermost first
            const uint32_t dt = r.get<uint32_t>();
            if (!dtype_block_size((int)dt)) bail("unknown dtype for tensor %u", dt);
            ti.ggml_dtype = (int)dt;
            ti.offset = r.get<uint64_t>();
            unsigned __int128 elems = 1;
            for (uint64_t d : ti.dims) {
                elems *= d;
                if (elems > (unsigned __int128)UINT64_MAX) bail("gguf: tensor %s has too many elements", ti.name.c_str());
            }
            ti.nbytes = (uint64_t)elems / dtype_block_size((int)dt) * dtype_type_size((int)dt);
            auto it = f->tensor_index.find(ti.name);
            if (it != f->tensor_index.end()) {
                f->tensors[it->second] = std::move(ti);
            } else {
                f->tensor_index.emplace(ti.name, f->tensors.size());
                f->tensors.push_back(std::move(ti));
            }
        }
        // general.alignment as an unsigned or non-negative signed 8/16/32-bit
        // value, otherwise the default of 32 (gguf.rs:445-454)
        uint64_t align = 32;
        auto it = f->meta_index.find("general.alignment");
        if (it != f->meta_index.end()) {
            const Value& v = f->metadata[it->second].second;
            if (v.type == VT_U8 || v.type == VT_U16 || v.type == VT_U32) align = v.u;
            else if ((v.type == VT_I8 || v.type == VT_I16 || v.type == VT_I32) && v.i >= 0) align = (uint64_t)v.i;
        }
        if (align == 0) bail("gguf: general.alignment is 0");
        f->tensor_data_offset = (r.pos + align - 1) / align * align;
    } catch (const ParseError& e) {
        err = e.what();
        return nullptr;
    } catch (const std::bad_alloc&) {
        err = "gguf: out of host memory while parsing the header";
        return nullptr;
    }
    return f;
}

}  // namespace gguf
}  // namespace frq

// safetensors.cpp -- checkpoint parsing (shared), the host FP32 loader of the
// reference API, and the streaming device loader.
//
// Format rules and error messages follow src/io/safetensors.cpp:237-608: the
// header is an 8-byte little-endian length (2 .. 100 MiB) and a UTF-8 JSON
// object whose keys are tensor names (or "__metadata__", a string-to-string
// object); a tensor is {"dtype", "shape", "data_offsets"} and nothing else;
// integers are non-negative without leading zeros; tensors must tile the
// payload exactly.
#include "stratakv/io/safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <functional>
#include <limits>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string_view>
#include <thread>
#include <unordered_set>
#include <vector>

#include "abi_check.h"

namespace stratakv {
namespace io {
namespace {

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

std::mutex g_breakdown_mutex;
LoadBreakdown g_breakdown;

void publish(const LoadBreakdown& b) {
    std::lock_guard<std::mutex> lock(g_breakdown_mutex);
    g_breakdown = b;
}

[[noreturn]] void fail(const std::string& why) { throw std::runtime_error("safetensors: " + why); }

constexpr std::uint64_t kMaxHeaderBytes = 100ull * 1024ull * 1024ull;

std::uint64_t le64(const unsigned char* p) {
    std::uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

// ---------------------------------------------------------------------------
// Header text checks and the schema-directed reader.
// ---------------------------------------------------------------------------
void check_utf8(std::string_view s) {
    std::size_t i = 0;
    while (i < s.size()) {
        const auto lead = static_cast<unsigned char>(s[i++]);
        if (lead < 0x80) continue;
        int follow;
        std::uint32_t cp, lowest;
        if (lead >= 0xC2 && lead <= 0xDF) {
            follow = 1, cp = lead & 0x1Fu, lowest = 0x80;
        } else if (lead >= 0xE0 && lead <= 0xEF) {
            follow = 2, cp = lead & 0x0Fu, lowest = 0x800;
        } else if (lead >= 0xF0 && lead <= 0xF4) {
            follow = 3, cp = lead & 0x07u, lowest = 0x10000;
        } else {
            fail("invalid UTF-8");
        }
        if (static_cast<std::size_t>(follow) > s.size() - i) fail("truncated UTF-8");
        for (; follow > 0; --follow) {
            const auto c = static_cast<unsigned char>(s[i++]);
            if ((c & 0xC0u) != 0x80u) fail("invalid UTF-8 continuation");
            cp = (cp << 6) | (c & 0x3Fu);
        }
        const bool surrogate = cp >= 0xD800 && cp <= 0xDFFF;
        if (cp < lowest || cp > 0x10FFFF || surrogate) fail("invalid UTF-8 codepoint");
    }
}

void put_utf8(std::string& out, std::uint32_t cp) {
    if (cp < 0x80) {
        out += static_cast<char>(cp);
    } else if (cp < 0x800) {
        out += static_cast<char>(0xC0u | (cp >> 6));
        out += static_cast<char>(0x80u | (cp & 0x3Fu));
    } else if (cp < 0x10000) {
        out += static_cast<char>(0xE0u | (cp >> 12));
        out += static_cast<char>(0x80u | ((cp >> 6) & 0x3Fu));
        out += static_cast<char>(0x80u | (cp & 0x3Fu));
    } else {
        out += static_cast<char>(0xF0u | (cp >> 18));
        out += static_cast<char>(0x80u | ((cp >> 12) & 0x3Fu));
        out += static_cast<char>(0x80u | ((cp >> 6) & 0x3Fu));
        out += static_cast<char>(0x80u | (cp & 0x3Fu));
    }
}

struct TensorSpec {
    std::string name;
    std::string dtype;
    std::vector<std::size_t> shape;
    std::size_t begin = 0, end = 0, count = 0;
};

class HeaderReader {
public:
    explicit HeaderReader(std::string_view text) : s_(text) {}

    std::vector<TensorSpec> read() {
        check_utf8(s_);
        if (s_.empty() || s_.front() != '{') fail("header must start with '{'");
        require('{');
        std::vector<TensorSpec> specs;
        std::unordered_set<std::string> seen;
        if (!accept('}')) {
            for (;;) {
                std::string key = str();
                if (!seen.insert(key).second) fail("duplicate top-level key");
                require(':');
                if (key == "__metadata__") metadata_object();
                else specs.push_back(tensor_object(std::move(key)));
                if (accept('}')) break;
                require(',');
            }
        }
        skip_ws();
        if (at_ != s_.size()) fail("trailing JSON data");
        return specs;
    }

private:
    void skip_ws() {
        while (at_ < s_.size()) {
            const char c = s_[at_];
            if (c != ' ' && c != '\t' && c != '\n' && c != '\r') break;
            ++at_;
        }
    }
    bool accept(char c) {
        skip_ws();
        if (at_ < s_.size() && s_[at_] == c) {
            ++at_;
            return true;
        }
        return false;
    }
    void require(char c) {
        if (!accept(c)) fail(std::string("expected '") + c + "' at header byte " + std::to_string(at_));
    }
    std::uint32_t hex4() {
        std::uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            if (at_ == s_.size()) fail("truncated unicode escape");
            const char c = s_[at_++];
            std::uint32_t d;
            if (c >= '0' && c <= '9') d = static_cast<std::uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') d = static_cast<std::uint32_t>(c - 'a') + 10u;
            else if (c >= 'A' && c <= 'F') d = static_cast<std::uint32_t>(c - 'A') + 10u;
            else fail("invalid unicode escape");
            v = v * 16u + d;
        }
        return v;
    }
    std::string str() {
        require('"');
        std::string out;
        while (at_ < s_.size()) {
            const auto c = static_cast<unsigned char>(s_[at_++]);
            if (c == '"') return out;
            if (c < 0x20) fail("unescaped control character");
            if (c != '\\') {
                out += static_cast<char>(c);
                continue;
            }
            if (at_ == s_.size()) fail("truncated string escape");
            const char e = s_[at_++];
            switch (e) {
            case '"': case '\\': case '/': out += e; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                std::uint32_t cp = hex4();
                if (cp >= 0xDC00 && cp <= 0xDFFF) fail("unpaired low surrogate");
                if (cp >= 0xD800 && cp <= 0xDBFF) {
                    if (s_.size() - at_ < 2 || s_[at_] != '\\' || s_[at_ + 1] != 'u')
                        fail("missing low surrogate");
                    at_ += 2;
                    const std::uint32_t lo = hex4();
                    if (lo < 0xDC00 || lo > 0xDFFF) fail("invalid low surrogate");
                    cp = 0x10000u + ((cp - 0xD800u) << 10) + (lo - 0xDC00u);
                }
                put_utf8(out, cp);
                break;
            }
            default: fail("invalid string escape");
            }
        }
        fail("unterminated string");
    }
    std::size_t uint() {
        skip_ws();
        const std::size_t start = at_;
        constexpr std::size_t kMax = std::numeric_limits<std::size_t>::max();
        std::size_t v = 0;
        while (at_ < s_.size() && s_[at_] >= '0' && s_[at_] <= '9') {
            const auto d = static_cast<std::size_t>(s_[at_++] - '0');
            if (v > (kMax - d) / 10) fail("integer overflow");
            v = v * 10 + d;
        }
        const bool none = at_ == start;
        if (none || (s_[start] == '0' && at_ - start > 1))
            fail("expected nonnegative JSON integer without leading zeros");
        return v;
    }
    std::vector<std::size_t> uint_list(std::size_t most) {
        require('[');
        std::vector<std::size_t> v;
        if (accept(']')) return v;
        for (;;) {
            if (v.size() == most) fail("array/rank limit exceeded");
            v.push_back(uint());
            if (accept(']')) return v;
            require(',');
        }
    }
    void metadata_object() {
        require('{');
        std::unordered_set<std::string> keys;
        if (accept('}')) return;
        for (;;) {
            if (!keys.insert(str()).second) fail("duplicate metadata key");
            require(':');
            (void)str();  // values must be strings
            if (accept('}')) return;
            require(',');
        }
    }
    TensorSpec tensor_object(std::string name) {
        TensorSpec t;
        t.name = std::move(name);
        require('{');
        if (accept('}')) fail("missing tensor fields");
        enum : unsigned { kDtype = 1, kShape = 2, kOffsets = 4 };
        unsigned have = 0;
        for (;;) {
            const std::string field = str();
            require(':');
            unsigned bit;
            if (field == "dtype") bit = kDtype;
            else if (field == "shape") bit = kShape;
            else if (field == "data_offsets") bit = kOffsets;
            else fail("unknown tensor field: " + field);
            if (have & bit) fail("duplicate tensor field: " + field);
            have |= bit;
            if (bit == kDtype) {
                t.dtype = str();
            } else if (bit == kShape) {
                t.shape = uint_list(64);
            } else {
                const auto off = uint_list(2);
                if (off.size() != 2) fail("data_offsets must contain two integers");
                t.begin = off[0];
                t.end = off[1];
            }
            if (accept('}')) break;
            require(',');
        }
        if (have != (kDtype | kShape | kOffsets)) fail("missing tensor fields");
        return t;
    }

    std::string_view s_;
    std::size_t at_ = 0;
};

std::size_t width_of(const std::string& dtype) { return dtype == "F32" ? 4u : 2u; }

// Element counts, byte ranges, and that the tensors tile the payload;
// returns the specs sorted by offset.
void check_specs(std::vector<TensorSpec>& specs, std::size_t payload) {
    constexpr auto kMaxBytes = static_cast<std::size_t>(std::numeric_limits<std::ptrdiff_t>::max());
    for (auto& t : specs) {
        if (t.dtype != "F32" && t.dtype != "F16" && t.dtype != "BF16" && t.dtype != "bfloat16")
            fail("unsupported dtype: " + t.dtype);
        const std::size_t w = width_of(t.dtype);
        const std::size_t most = kMaxBytes / w;
        std::size_t n = 1;
        for (auto d = t.shape.rbegin(); d != t.shape.rend(); ++d) {
            if (*d != 0 && n > most / *d) fail("tensor shape overflow");
            n *= *d;
        }
        t.count = n;
        if (t.begin > t.end || t.end > payload || t.end - t.begin != n * w)
            fail("invalid tensor byte range: " + t.name);
    }
    std::sort(specs.begin(), specs.end(), [](const TensorSpec& a, const TensorSpec& b) {
        return a.begin != b.begin ? a.begin < b.begin : a.end < b.end;
    });
    std::size_t next = 0;
    for (const auto& t : specs) {
        if (t.begin != next) fail("overlapping tensors or hole in payload");
        next = t.end;
    }
    if (next != payload) fail("unreferenced/truncated payload");
}

// ---------------------------------------------------------------------------
// File access.
// ---------------------------------------------------------------------------
struct OpenFile {
    int fd = -1;
    std::size_t size = 0;
    ~OpenFile() {
        if (fd >= 0) ::close(fd);
    }
};

std::unique_ptr<OpenFile> open_file(const std::filesystem::path& path) {
    auto f = std::make_unique<OpenFile>();
    f->fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) fail("open failed: errno=" + std::to_string(errno));
    struct stat st {};
    if (::fstat(f->fd, &st) != 0 || !S_ISREG(st.st_mode) || st.st_size < 0)
        fail("fstat failed or file is not regular");
    const auto len = static_cast<std::uintmax_t>(st.st_size);
    if (len < 8 || len > static_cast<std::uintmax_t>(std::numeric_limits<std::ptrdiff_t>::max()))
        fail("file too small or too large for this address space");
    f->size = static_cast<std::size_t>(len);
    return f;
}

void read_exact(int fd, void* dst, std::size_t bytes, std::size_t offset) {
    auto* p = static_cast<unsigned char*>(dst);
    while (bytes > 0) {
        const ssize_t got = ::pread(fd, p, bytes, static_cast<off_t>(offset));
        if (got < 0) {
            if (errno == EINTR) continue;
            fail("read failed: errno=" + std::to_string(errno));
        }
        if (got == 0) fail("read failed: unexpected end of file");
        p += got;
        offset += static_cast<std::size_t>(got);
        bytes -= static_cast<std::size_t>(got);
    }
}

// Header length, text and validated specs of an open file.
std::vector<TensorSpec> read_header(const unsigned char* first8, const std::function<std::string(std::size_t)>& text_of,
                                    std::size_t file_size, std::size_t* data_start) {
    const std::uint64_t hlen = le64(first8);
    if (hlen < 2 || hlen > kMaxHeaderBytes || hlen > file_size - 8) fail("invalid or oversized header length");
    const std::string text = text_of(static_cast<std::size_t>(hlen));
    auto specs = HeaderReader(text).read();
    *data_start = 8 + static_cast<std::size_t>(hlen);
    check_specs(specs, file_size - *data_start);
    return specs;
}

bool is_norm_name(const std::string& n) {
    for (const char* k : {"norm", "Norm", "gamma", "Gamma"})
        if (n.find(k) != std::string::npos) return true;
    return false;
}

std::uint32_t half_bits_to_f32(std::uint16_t h) {
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const std::uint32_t exp = (h >> 10) & 0x1Fu;
    std::uint32_t mant = h & 0x3FFu;
    if (exp == 0x1Fu) return sign | 0x7F800000u | (mant << 13);
    if (exp != 0) return sign | ((exp + 112u) << 23) | (mant << 13);
    if (mant == 0) return sign;
    int e = 113;  // biased exponent of 2^-14 plus one normalisation step
    do {
        mant <<= 1;
        --e;
    } while ((mant & 0x400u) == 0);
    return sign | (static_cast<std::uint32_t>(e) << 23) | ((mant & 0x3FFu) << 13);
}

struct Mapping {
    void* base = MAP_FAILED;
    std::size_t size = 0;
    ~Mapping() {
        if (base != MAP_FAILED) ::munmap(base, size);
    }
};

// Runs body(begin, end) over [0, n) on up to `threads` threads.
template <typename F>
void split_run(std::size_t n, unsigned threads, std::size_t min_per_thread, F body) {
    const std::size_t want = std::max<std::size_t>(1, std::min<std::size_t>(threads, n / std::max<std::size_t>(min_per_thread, 1)));
    if (want <= 1) {
        body(std::size_t{0}, n);
        return;
    }
    std::vector<std::thread> pool;
    std::exception_ptr error;
    std::mutex error_mutex;
    const std::size_t step = (n + want - 1) / want;
    for (std::size_t b = 0; b < n; b += step) {
        const std::size_t e = std::min(n, b + step);
        pool.emplace_back([&, b, e] {
            try {
                body(b, e);
            } catch (...) {
                std::lock_guard<std::mutex> lock(error_mutex);
                if (!error) error = std::current_exception();
            }
        });
    }
    for (auto& t : pool) t.join();
    if (error) std::rethrow_exception(error);
}

unsigned worker_count() {
    const unsigned hw = std::thread::hardware_concurrency();
    return std::max(1u, std::min(8u, hw));
}

}  // namespace

LoadBreakdown last_load_breakdown() noexcept {
    std::lock_guard<std::mutex> lock(g_breakdown_mutex);
    return g_breakdown;
}

// ---------------------------------------------------------------------------
// Host FP32 loader (reference API).
// ---------------------------------------------------------------------------
WeightMap load_safetensors(const std::filesystem::path& path, bool require_mapped_f32) {
    LoadBreakdown bd;
    auto t0 = Clock::now();
    auto file = open_file(path);
    auto map = std::make_shared<Mapping>();
    map->size = file->size;
    // Private writable mapping: FP32 aliases are handed out as float*.
    map->base = ::mmap(nullptr, file->size, PROT_READ | PROT_WRITE, MAP_PRIVATE, file->fd, 0);
    if (map->base == MAP_FAILED) fail("mmap failed: errno=" + std::to_string(errno));
    bd.mmap_open_ms = ms_since(t0);
    const auto* bytes = static_cast<const unsigned char*>(map->base);

    t0 = Clock::now();
    std::size_t data_start = 0;
    auto specs = read_header(
        bytes, [&](std::size_t n) { return std::string(reinterpret_cast<const char*>(bytes) + 8, n); },
        file->size, &data_start);
    bd.header_parse_ms = ms_since(t0);

    t0 = Clock::now();
    WeightMap out;
    out.reserve(specs.size());
    for (const auto& t : specs) {
        const unsigned char* src = bytes + data_start + t.begin;
        const bool f32 = t.dtype == "F32";
        const bool alias = f32 && is_norm_name(t.name) && t.count != 0 &&
                           reinterpret_cast<std::uintptr_t>(src) % 64 == 0;
        if (require_mapped_f32 && f32 && t.count != 0 && !alias)
            fail("F32 tensor is not directly mappable: " + t.name);
        if (alias) {
            out.emplace(t.name, Tensor::from_external(t.shape, reinterpret_cast<float*>(const_cast<unsigned char*>(src)),
                                                      std::shared_ptr<void>(map, map->base)));
            continue;
        }
        Tensor dst(t.shape, DataType::FP32, Device::CPU);
        auto* d = static_cast<std::uint32_t*>(dst.raw_data());
        const std::string dtype = t.dtype;
        split_run(t.count, worker_count(), std::size_t{1} << 20, [&](std::size_t b, std::size_t e) {
            for (std::size_t i = b; i < e; ++i) {
                if (dtype == "F32") {
                    std::uint32_t v;
                    std::memcpy(&v, src + 4 * i, 4);  // little-endian host
                    d[i] = v;
                } else {
                    const auto h = static_cast<std::uint16_t>(src[2 * i] | (src[2 * i + 1] << 8));
                    d[i] = dtype == "F16" ? half_bits_to_f32(h) : static_cast<std::uint32_t>(h) << 16;
                }
            }
        });
        out.emplace(t.name, std::move(dst));
        bd.payload_bytes += t.end - t.begin;
    }
    bd.tensor_decode_ms = ms_since(t0);
    publish(bd);
    return out;
}

// ---------------------------------------------------------------------------
// Device loader: pread into page-locked chunks (several threads), async copy
// to HBM while the next chunk is read; F16 widened on the device.
// ---------------------------------------------------------------------------
namespace {

constexpr std::size_t kChunkBytes = 64u << 20;
constexpr int kRing = 2;

struct StagingRing {
    void* host[kRing] = {};
    void* dev[kRing] = {};
    void* done[kRing] = {};   // event: last copy out of host[k] finished
    bool pending[kRing] = {};
    ~StagingRing() {
        for (int k = 0; k < kRing; ++k) {
            if (done[k]) {
                if (pending[k]) (void)skv_event_synchronize(done[k]);
                (void)skv_event_destroy(done[k]);
            }
            if (host[k]) (void)skv_host_free(host[k]);
            if (dev[k]) (void)skv_free(dev[k]);
        }
    }
};

}  // namespace

WeightMap load_safetensors_device(const std::filesystem::path& path, void* stream) {
    LoadBreakdown bd;
    auto t0 = Clock::now();
    auto file = open_file(path);
    bd.mmap_open_ms = ms_since(t0);

    t0 = Clock::now();
    unsigned char first8[8];
    read_exact(file->fd, first8, 8, 0);
    std::size_t data_start = 0;
    auto specs = read_header(
        first8,
        [&](std::size_t n) {
            std::string s(n, '\0');
            read_exact(file->fd, s.data(), n, 8);
            return s;
        },
        file->size, &data_start);
    bd.header_parse_ms = ms_since(t0);

    t0 = Clock::now();
    WeightMap out;
    out.reserve(specs.size());
    StagingRing ring;
    const bool any_f16 = std::any_of(specs.begin(), specs.end(), [](const TensorSpec& t) { return t.dtype == "F16"; });
    for (int k = 0; k < kRing; ++k) {
        detail::check(skv_host_alloc(&ring.host[k], kChunkBytes), "load_safetensors_device: staging");
        detail::check(skv_event_create(&ring.done[k]), "load_safetensors_device: staging");
        if (any_f16) detail::check(skv_malloc(&ring.dev[k], kChunkBytes), "load_safetensors_device: staging");
    }
    // Every destination is allocated before the first copy is queued, so no
    // allocation waits on copies in flight.
    std::vector<Tensor> dsts;
    dsts.reserve(specs.size());
    for (const auto& t : specs) {
        const bool bf16 = t.dtype == "BF16" || t.dtype == "bfloat16";
        dsts.emplace_back(t.shape, bf16 ? DataType::BF16 : DataType::FP32, Device::GPU);
    }
    int slot = 0;
    const unsigned threads = worker_count();
    for (std::size_t ti = 0; ti < specs.size(); ++ti) {
        const auto& t = specs[ti];
        const bool f16 = t.dtype == "F16";
        Tensor& dst = dsts[ti];
        auto* dbase = static_cast<unsigned char*>(dst.raw_data());
        const std::size_t total = t.end - t.begin;
        for (std::size_t off = 0; off < total; off += kChunkBytes) {
            const std::size_t n = std::min(kChunkBytes, total - off);
            if (ring.pending[slot]) {
                detail::check(skv_event_synchronize(ring.done[slot]), "load_safetensors_device: copy");
                ring.pending[slot] = false;
            }
            auto* h = static_cast<unsigned char*>(ring.host[slot]);
            const std::size_t file_off = data_start + t.begin + off;
            split_run(n, threads, std::size_t{4} << 20, [&](std::size_t b, std::size_t e) {
                read_exact(file->fd, h + b, e - b, file_off + b);
            });
            if (f16) {
                detail::check(skv_memcpy_h2d_async(ring.dev[slot], h, n, stream), "load_safetensors_device: copy");
                detail::check(skv_convert_to_f32(ring.dev[slot], SKV_DTYPE_F16, n / 2,
                                                 reinterpret_cast<float*>(dbase + off * 2), nullptr, stream),
                              "load_safetensors_device: F16 widening");
            } else {
                detail::check(skv_memcpy_h2d_async(dbase + off, h, n, stream), "load_safetensors_device: copy");
            }
            detail::check(skv_event_record(ring.done[slot], stream), "load_safetensors_device: copy");
            ring.pending[slot] = true;
            slot = (slot + 1) % kRing;
        }
        bd.payload_bytes += total;
    }
    detail::check(skv_stream_synchronize(stream), "load_safetensors_device: copy");
    for (std::size_t ti = 0; ti < specs.size(); ++ti) out.emplace(specs[ti].name, std::move(dsts[ti]));
    for (int k = 0; k < kRing; ++k) ring.pending[k] = false;
    bd.tensor_decode_ms = ms_since(t0);
    publish(bd);
    return out;
}

Tensor load_linear_bf16_transposed(const Tensor& source, std::size_t out_features, std::size_t in_features) {
    if (source.ndim() != 2 || source.shape() != std::vector<std::size_t>{out_features, in_features} ||
        (source.dtype() != DataType::BF16 && source.dtype() != DataType::FP32) ||
        source.device() != Device::CPU)
        throw std::invalid_argument("safetensors: expected a BF16 or FP32 [out, in] linear tensor");
    Tensor dst({in_features, out_features}, DataType::BF16, Device::CPU);
    auto* d = static_cast<std::uint16_t*>(dst.raw_data());
    const auto& st = source.strides();
    const bool bf16 = source.dtype() == DataType::BF16;
    const auto* s16 = static_cast<const std::uint16_t*>(source.raw_data());
    const auto* s32 = static_cast<const std::uint32_t*>(source.raw_data());
    constexpr std::size_t kTile = 64;
    split_run((out_features + kTile - 1) / kTile, worker_count(), 1, [&](std::size_t tb, std::size_t te) {
        for (std::size_t to = tb * kTile; to < std::min(out_features, te * kTile); to += kTile)
            for (std::size_t ti = 0; ti < in_features; ti += kTile)
                for (std::size_t o = to; o < std::min(out_features, to + kTile); ++o)
                    for (std::size_t i = ti; i < std::min(in_features, ti + kTile); ++i) {
                        const std::size_t si = o * st[0] + i * st[1];
                        d[i * out_features + o] = bf16 ? s16[si] : static_cast<std::uint16_t>(s32[si] >> 16);
                    }
    });
    return dst;
}

}  // namespace io
}  // namespace stratakv

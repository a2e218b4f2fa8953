// Safetensors checkpoints: every shard is memory-mapped read-only; its header (8-byte
// little-endian length, then a JSON object name -> {dtype, shape, data_offsets}) is turned
// into one Entry per tensor, checked against the shard before it is accepted:
//   * the header must fit the file, the JSON must be one object of objects;
//   * a tensor's byte range must lie inside the shard's data section;
//   * a tensor of a known dtype must hold exactly numel x element-size bytes.
// Tensor bytes are never copied: views and the device upload read the mapping.
#include "safetensors_loader.h"

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <iostream>

namespace {

// Bytes per element of the dtypes a checkpoint may hold (0: unknown to this reader).
size_t dtype_size(const std::string& dt) {
    if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
    if (dt == "BF16" || dt == "F16" || dt == "I16" || dt == "U16") return 2;
    if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
    if (dt == "I8" || dt == "U8" || dt == "BOOL" || dt == "F8_E4M3" || dt == "F8_E5M2") return 1;
    return 0;
}

// n elements of a BF16 or F32 tensor as fp32 (bf16 is the upper half of an fp32: exact).
bool widen(const std::string& dt, const void* src, int64_t n, float* dst) {
    if (dt == "F32") {
        // (no copy of an empty tensor: dst may then be null; a shape-less entry has 0
        // elements, as numel() defines it)
        if (n > 0) std::memcpy(dst, src, static_cast<size_t>(n) * 4);
        return true;
    }
    if (dt == "BF16") {
        const auto* h = static_cast<const uint16_t*>(src);
        for (int64_t i = 0; i < n; ++i) dst[i] = bf16_to_f32(h[i]);
        return true;
    }
    return false;
}

// Tokens of the header JSON, enough for its grammar: objects, arrays, strings, integers,
// and literals (true / false / null / other numbers) skipped as a whole.
class Json {
public:
    Json(const char* begin, const char* end) : p_(begin), end_(end) {}
    bool failed() const { return bad_; }

    // Consumes `c` (after white space); false when the next character differs.
    bool eat(char c) {
        blank();
        if (p_ < end_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) bad_ = true;
    }
    std::string string() {
        std::string s;
        if (!eat('"')) {
            bad_ = true;
            return s;
        }
        for (; p_ < end_ && *p_ != '"'; ++p_) {
            if (*p_ != '\\') {
                s.push_back(*p_);
                continue;
            }
            if (++p_ >= end_) break;
            switch (*p_) {
                case 'n': s.push_back('\n'); break;
                case 't': s.push_back('\t'); break;
                case 'r': s.push_back('\r'); break;
                case 'b': s.push_back('\b'); break;
                case 'f': s.push_back('\f'); break;
                default: s.push_back(*p_); break;  // \" \\ \/ (and \u.... kept as written)
            }
        }
        if (p_ >= end_) {
            bad_ = true;
            return s;
        }
        ++p_;  // closing quote
        return s;
    }
    int64_t integer() {
        blank();
        bool neg = false;
        if (p_ < end_ && (*p_ == '-' || *p_ == '+')) neg = *p_++ == '-';
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') {
            bad_ = true;
            return 0;
        }
        int64_t v = 0;
        for (; p_ < end_ && *p_ >= '0' && *p_ <= '9'; ++p_) {
            if (v > (INT64_MAX - (*p_ - '0')) / 10) {
                bad_ = true;
                return 0;
            }
            v = v * 10 + (*p_ - '0');
        }
        return neg ? -v : v;
    }
    std::vector<int64_t> integers() {
        std::vector<int64_t> v;
        expect('[');
        if (eat(']')) return v;
        do v.push_back(integer());
        while (!bad_ && eat(','));
        expect(']');
        return v;
    }
    // Skips one value of any kind.
    void value() {
        blank();
        if (p_ >= end_) {
            bad_ = true;
            return;
        }
        if (*p_ == '"') {
            string();
        } else if (*p_ == '{' || *p_ == '[') {
            const bool obj = *p_ == '{';
            ++p_;
            if (eat(obj ? '}' : ']')) return;
            do {
                if (obj) {
                    string();
                    expect(':');
                }
                value();
            } while (!bad_ && eat(','));
            expect(obj ? '}' : ']');
        } else {
            const char* start = p_;
            while (p_ < end_ && !std::strchr(",}] \t\r\n", *p_)) ++p_;
            if (p_ == start) bad_ = true;
        }
    }

private:
    void blank() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    const char* p_;
    const char* end_;
    bool bad_ = false;
};

bool complain(const std::string& where, const std::string& what) {
    std::cerr << "[safetensors] " << where << ": " << what << "\n";
    return false;
}

}  // namespace

int64_t SafeTensors::Entry::numel() const {
    if (shape.empty()) return 0;
    int64_t n = 1;
    for (const int64_t d : shape) n *= d;
    return n;
}

SafeTensors::~SafeTensors() { release(); }

void SafeTensors::release() {
    for (const Shard& s : shards_) munmap(s.map, s.size);
    shards_.clear();
    entries_.clear();
    f32_cache_.clear();
}

bool SafeTensors::parse_shard(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return complain(path, "cannot be opened");
    struct stat sb {};
    if (::fstat(fd, &sb) != 0 || sb.st_size < 8) {
        ::close(fd);
        return complain(path, "shorter than the 8-byte header length");
    }
    const size_t size = static_cast<size_t>(sb.st_size);
    void* map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED) return complain(path, "cannot be mapped");
    shards_.push_back({map, size});
    const int shard = static_cast<int>(shards_.size()) - 1;
    const char* base = static_cast<const char*>(map);

    uint64_t hlen = 0;
    std::memcpy(&hlen, base, 8);
    if (hlen > size - 8)
        return complain(path, "a header of " + std::to_string(hlen) + " bytes does not fit a file of " +
                                  std::to_string(size) + " bytes");
    const size_t data0 = 8 + static_cast<size_t>(hlen), data_bytes = size - data0;

    std::vector<std::pair<std::string, Entry>> found;
    Json js(base + 8, base + data0);
    js.expect('{');
    if (!js.failed() && !js.eat('}')) {
        do {
            std::string name = js.string();
            js.expect(':');
            if (js.failed()) break;
            if (name == "__metadata__") {
                js.value();
                continue;
            }
            Entry e;
            std::vector<int64_t> span;
            js.expect('{');
            if (!js.eat('}')) {
                do {
                    const std::string field = js.string();
                    js.expect(':');
                    if (field == "dtype") e.dtype = js.string();
                    else if (field == "shape") e.shape = js.integers();
                    else if (field == "data_offsets") span = js.integers();
                    else js.value();
                } while (!js.failed() && js.eat(','));
                js.expect('}');
            }
            if (js.failed()) break;
            if (span.size() != 2 || span[0] < 0 || span[1] < span[0] || static_cast<uint64_t>(span[1]) > data_bytes)
                return complain(path, "tensor '" + name + "' does not lie inside the " + std::to_string(data_bytes) +
                                          "-byte data section");
            for (const int64_t d : e.shape)
                if (d < 0) return complain(path, "tensor '" + name + "' has a negative dimension");
            e.shard = shard;
            e.abs_offset = data0 + static_cast<size_t>(span[0]);
            e.nbytes = static_cast<size_t>(span[1] - span[0]);
            const size_t es = dtype_size(e.dtype);
            // the element count in checked arithmetic: a shape whose product (or its byte size)
            // wraps around could otherwise equal the span and pass the check below
            int64_t count = 1, bytes = 0;
            bool wraps = false;
            for (const int64_t d : e.shape) wraps = wraps || __builtin_mul_overflow(count, d, &count);
            wraps = wraps || __builtin_mul_overflow(count, static_cast<int64_t>(es), &bytes);
            if (wraps)
                return complain(path, "tensor '" + name + "' has a shape whose size overflows 64 bits");
            if (es && static_cast<size_t>(e.numel()) * es != e.nbytes && !e.shape.empty())
                return complain(path, "tensor '" + name + "' holds " + std::to_string(e.nbytes) + " bytes, not " +
                                          std::to_string(e.numel()) + " x " + std::to_string(es));
            found.emplace_back(std::move(name), std::move(e));
        } while (!js.failed() && js.eat(','));
        js.expect('}');
    }
    if (js.failed()) return complain(path, "the JSON header is malformed");
    for (auto& kv : found) entries_[kv.first] = std::move(kv.second);
    std::cerr << "[safetensors] shard '" << path << "': " << (size >> 20) << " MB\n";
    return true;
}

bool SafeTensors::load(const std::string& path) {
    release();
    return parse_shard(path);
}

bool SafeTensors::load_model(const std::string& model_dir) {
    release();
    std::vector<std::string> shard_files;
    if (DIR* dir = ::opendir(model_dir.c_str())) {
        const std::string suffix = ".safetensors";
        while (const dirent* de = ::readdir(dir)) {
            const std::string f = de->d_name;
            if (f.size() > suffix.size() && f.compare(f.size() - suffix.size(), suffix.size(), suffix) == 0)
                shard_files.push_back(model_dir + "/" + f);
        }
        ::closedir(dir);
    }
    if (shard_files.empty()) return complain(model_dir, "holds no *.safetensors shard");
    std::sort(shard_files.begin(), shard_files.end());
    for (const std::string& f : shard_files)
        if (!parse_shard(f)) return false;
    std::cerr << "[safetensors] " << shard_files.size() << " shard(s), " << entries_.size() << " tensors\n";
    return true;
}

const SafeTensors::Entry* SafeTensors::find(const std::string& name) const {
    const auto it = entries_.find(name);
    return it != entries_.end() ? &it->second : nullptr;
}

const void* SafeTensors::data(const std::string& name) const {
    const Entry* e = find(name);
    return e ? static_cast<const uint8_t*>(shards_[static_cast<size_t>(e->shard)].map) + e->abs_offset : nullptr;
}

WeightView SafeTensors::view(const std::string& name) const {
    WeightView v;
    if (const Entry* e = find(name)) {
        v.numel = e->numel();
        if (e->dtype == "BF16") v.bf16 = static_cast<const uint16_t*>(data(name));
        if (e->dtype == "F32") v.f32 = static_cast<const float*>(data(name));
    }
    return v;
}

const float* SafeTensors::get_f32(const std::string& name, int64_t* out_numel) {
    auto cached = f32_cache_.find(name);
    if (cached == f32_cache_.end()) {
        const Entry* e = find(name);
        if (!e) return nullptr;
        std::vector<float> wide(static_cast<size_t>(e->numel()));
        if (!widen(e->dtype, data(name), e->numel(), wide.data())) {
            complain(name, "dtype " + e->dtype + " cannot be widened to fp32");
            return nullptr;
        }
        cached = f32_cache_.emplace(name, std::move(wide)).first;
    }
    if (out_numel) *out_numel = static_cast<int64_t>(cached->second.size());
    return cached->second.data();
}

bool SafeTensors::get_row_f32(const std::string& name, int64_t row, float* dst) const {
    const Entry* e = find(name);
    if (!e || e->shape.size() != 2 || row < 0 || row >= e->shape[0]) return false;
    const int64_t width = e->shape[1];
    const size_t es = dtype_size(e->dtype);
    const auto* first = static_cast<const uint8_t*>(data(name)) + static_cast<size_t>(row * width) * es;
    return es != 0 && widen(e->dtype, first, width, dst);
}

void SafeTensors::device_table(std::vector<q35_tensor>* out) const {
    out->clear();
    out->reserve(entries_.size());
    for (const auto& kv : entries_) {
        const Entry& e = kv.second;
        q35_tensor t{};
        t.name = kv.first.c_str();
        t.dtype = e.dtype == "BF16" ? 0 : e.dtype == "F32" ? 1 : 2;
        t.ndim = static_cast<int32_t>(std::min<size_t>(e.shape.size(), 4));
        for (int i = 0; i < t.ndim; ++i) t.shape[i] = e.shape[static_cast<size_t>(i)];
        t.data = data(kv.first);
        out->push_back(t);
    }
}

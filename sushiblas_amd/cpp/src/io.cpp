// io.cpp -- IO::save_npy / load_npy / save_bin / load_bin (src/io.cpp of the
// reference) on the HIP backend.  Format and deviations: io.hpp.
#include <SushiBLAS/engine.hpp>
#include <SushiBLAS/io.hpp>

#include <algorithm>
#include <cstring>

namespace SushiBLAS
{
    namespace
    {
        constexpr size_t kChunk = size_t(64) << 20;  // pinned staging buffer size

        void hip_check(hipError_t e, const char* what)
        {
            SB_THROW_IF(e != hipSuccess, "{} failed: {}", what, hipGetErrorString(e));
        }

        struct Pinned
        {
            void* p = nullptr;
            explicit Pinned(size_t bytes)
            {
                hip_check(hipHostMalloc(&p, bytes > 0 ? bytes : 1, hipHostMallocDefault),
                          "hipHostMalloc");
            }
            ~Pinned()
            {
                if (p) (void)hipHostFree(p);
            }
            char* bytes() const { return static_cast<char*>(p); }
        };

        // Waits for the stream on every exit path, so no copy still reads or
        // writes a staging buffer when it is freed.
        struct StreamDrain
        {
            hipStream_t s;
            ~StreamDrain() { (void)hipStreamSynchronize(s); }
        };

        struct File
        {
            std::FILE* f = nullptr;
            File(const std::string& path, const char* mode) : f(std::fopen(path.c_str(), mode)) {}
            ~File()
            {
                if (f) std::fclose(f);
            }
        };

        // Element offsets (in elements, from the view's first element) in file
        // order: C order (last index fastest) or Fortran order (first fastest).
        template <typename F>
        void for_each_offset(const Tensor& t, bool fortran, F&& fn)
        {
            const int r = t.rank;
            if (t.num_elements == 0) return;
            int64_t idx[Core::MAX_TENSOR_RANK] = {0};
            int64_t off = 0;
            for (int64_t e = 0; e < t.num_elements; ++e)
            {
                fn(e, off);
                // advance the multi-index in file order
                for (int q = 0; q < r; ++q)
                {
                    const int d = fortran ? q : r - 1 - q;
                    if (++idx[d] < t.shape[d])
                    {
                        off += t.strides[d];
                        break;
                    }
                    off -= (t.shape[d] - 1) * t.strides[d];
                    idx[d] = 0;
                }
            }
        }

        // Elements spanned by the view from its first element (strides >= 0).
        int64_t span_elements(const Tensor& t)
        {
            if (t.num_elements == 0) return 0;
            int64_t last = 0;
            for (int d = 0; d < t.rank; ++d) last += (t.shape[d] - 1) * t.strides[d];
            return last + 1;
        }

        bool file_order_matches(const Tensor& t, bool fortran)
        {
            if (!t.is_contiguous()) return false;
            int big = 0;  // dimensions longer than 1 decide the order
            for (int d = 0; d < t.rank; ++d) big += t.shape[d] > 1;
            if (big <= 1) return true;
            return (t.layout == Core::Layout::COLUMN_MAJOR) == fortran;
        }

        void write_all(std::FILE* f, const void* p, size_t n, const std::string& path)
        {
            SB_THROW_IF(n && std::fwrite(p, 1, n, f) != n, "Short write to {}", path);
        }

        void read_all(std::FILE* f, void* p, size_t n, const std::string& path)
        {
            SB_THROW_IF(n && std::fread(p, 1, n, f) != n, "File {} is truncated", path);
        }

        size_t skip_ws(const std::string& s, size_t i)
        {
            while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
            return i;
        }

        // Position just after "'key':" (either quote style), or npos.
        size_t after_key(const std::string& dict, const char* key)
        {
            for (const char q : {'\'', '"'})
            {
                const std::string k = std::string(1, q) + key + std::string(1, q);
                size_t p = dict.find(k);
                if (p == std::string::npos) continue;
                p = skip_ws(dict, p + k.size());
                if (p < dict.size() && dict[p] == ':') return skip_ws(dict, p + 1);
            }
            return std::string::npos;
        }
    } // namespace

    const char* IO::npy_descr(Core::DataType dtype)
    {
        switch (dtype)
        {
            case Core::DataType::HALF: return "<f2";
            case Core::DataType::FLOAT32: return "<f4";
            case Core::DataType::FLOAT64: return "<f8";
            case Core::DataType::COMPLEX32: return "<c8";
            case Core::DataType::COMPLEX64: return "<c16";
        }
        return "";
    }

    size_t IO::element_bytes(Core::DataType dtype)
    {
        switch (dtype)
        {
            case Core::DataType::HALF: return 2;
            case Core::DataType::FLOAT32: return 4;
            case Core::DataType::FLOAT64: return 8;
            case Core::DataType::COMPLEX32: return 8;
            case Core::DataType::COMPLEX64: return 16;
        }
        return 4;
    }

    std::string IO::npy_header(Core::DataType dtype, Core::Layout layout, const int64_t* shape,
                               int rank)
    {
        std::string dict = "{'descr': '";
        dict += npy_descr(dtype);
        dict += "', 'fortran_order': ";
        dict += layout == Core::Layout::COLUMN_MAJOR ? "True" : "False";
        dict += ", 'shape': (";
        for (int i = 0; i < rank; ++i)
        {
            dict += std::to_string(shape[i]);
            if (rank == 1 || i < rank - 1) dict += ",";
            if (i < rank - 1) dict += " ";
        }
        dict += "), }";
        // magic (6) + version (2) + length (2) + dict + '\n' on a 64-byte boundary
        const size_t pad = (64 - (10 + dict.size() + 1) % 64) % 64;
        dict.append(pad, ' ');
        dict += '\n';
        SB_THROW_IF(dict.size() > 65535, "npy header too long ({} bytes)", dict.size());
        std::string out("\x93NUMPY\x01\x00", 8);
        out += static_cast<char>(dict.size() & 0xff);
        out += static_cast<char>((dict.size() >> 8) & 0xff);
        return out + dict;
    }

    NpyHeader IO::parse_npy_header(const std::string& b)
    {
        SB_THROW_IF(b.size() < 10 || b.compare(0, 6, std::string("\x93NUMPY", 6)) != 0,
                    "Invalid .npy file magic.");
        const unsigned major = static_cast<unsigned char>(b[6]);
        size_t hlen, start;
        if (major == 1)
        {
            hlen = static_cast<unsigned char>(b[8]) | (size_t(static_cast<unsigned char>(b[9])) << 8);
            start = 10;
        }
        else
        {
            SB_THROW_IF(major != 2 && major != 3, "Unsupported .npy format version {}", major);
            SB_THROW_IF(b.size() < 12, "Truncated .npy header");
            hlen = 0;
            for (int i = 0; i < 4; ++i) hlen |= size_t(static_cast<unsigned char>(b[8 + i])) << (8 * i);
            start = 12;
        }
        SB_THROW_IF(b.size() < start + hlen, "Truncated .npy header");
        const std::string dict = b.substr(start, hlen);
        NpyHeader h;
        h.data_offset = start + hlen;

        size_t p = after_key(dict, "descr");
        SB_THROW_IF(p == std::string::npos || p >= dict.size(), "npy header has no descr");
        const char q = dict[p];
        SB_THROW_IF(q != '\'' && q != '"', "npy descr is not a string");
        const size_t e = dict.find(q, p + 1);
        SB_THROW_IF(e == std::string::npos, "npy descr is not terminated");
        h.descr = dict.substr(p + 1, e - p - 1);

        p = after_key(dict, "fortran_order");
        SB_THROW_IF(p == std::string::npos, "npy header has no fortran_order");
        if (dict.compare(p, 4, "True") == 0) h.fortran_order = true;
        else SB_THROW_IF(dict.compare(p, 5, "False") != 0, "npy fortran_order is not a bool");

        p = after_key(dict, "shape");
        SB_THROW_IF(p == std::string::npos || p >= dict.size() || dict[p] != '(',
                    "npy header has no shape tuple");
        const size_t close = dict.find(')', p);
        SB_THROW_IF(close == std::string::npos, "npy shape is not terminated");
        std::string item;
        for (size_t i = p + 1; i <= close; ++i)
        {
            const char c = dict[i];
            if (c == ',' || c == ')')
            {
                size_t a = skip_ws(item, 0), z = item.size();
                while (z > a && (item[z - 1] == ' ' || item[z - 1] == 'L')) --z;
                if (z > a)
                {
                    const std::string num = item.substr(a, z - a);
                    SB_THROW_IF(num.find_first_not_of("0123456789") != std::string::npos,
                                "npy shape entry '{}' is not a size", num);
                    h.shape.push_back(std::stoll(num));
                }
                item.clear();
            }
            else
            {
                item += c;
            }
        }
        return h;
    }

    void IO::write_elements(const Tensor& t, std::FILE* f, const std::string& path, bool fortran)
    {
        const size_t bpe = element_bytes(t.dtype);
        const size_t bytes = static_cast<size_t>(t.num_elements) * bpe;
        if (bytes == 0) return;
        const bool device = t.storage->strategy == SushiRuntime::Memory::AllocStrategy::DEVICE;
        if (file_order_matches(t, fortran))
        {
            if (!device)
            {
                write_all(f, t.data(), bytes, path);
                return;
            }
            // HBM -> pinned (async, chunk i+1) while chunk i goes to the file
            hipStream_t s = engine_.get_context().get_queue().native();
            const size_t chunk = std::min(kChunk, bytes);
            Pinned buf0(chunk), buf1(chunk);
            char* bufs[2] = {buf0.bytes(), buf1.bytes()};
            StreamDrain drain{s};
            const char* src = static_cast<const char*>(t.data());
            const size_t n_chunks = (bytes + chunk - 1) / chunk;
            auto issue = [&](size_t i) {
                const size_t off = i * chunk, n = std::min(chunk, bytes - off);
                hip_check(hipMemcpyAsync(bufs[i & 1], src + off, n, hipMemcpyDeviceToHost, s),
                          "hipMemcpyAsync(D2H)");
            };
            issue(0);
            for (size_t i = 0; i < n_chunks; ++i)
            {
                hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
                if (i + 1 < n_chunks) issue(i + 1);
                const size_t off = i * chunk, n = std::min(chunk, bytes - off);
                write_all(f, bufs[i & 1], n, path);
            }
            return;
        }
        // general view: gather in file order from a host copy of the span
        const size_t span = static_cast<size_t>(span_elements(t)) * bpe;
        std::vector<char> host;
        const char* base;
        if (device)
        {
            host.resize(span);
            hip_check(hipMemcpy(host.data(), t.data(), span, hipMemcpyDeviceToHost), "hipMemcpy(D2H)");
            base = host.data();
        }
        else
        {
            base = static_cast<const char*>(t.data());
        }
        std::vector<char> out(bytes);
        for_each_offset(t, fortran, [&](int64_t e, int64_t off) {
            std::memcpy(out.data() + e * bpe, base + off * bpe, bpe);
        });
        write_all(f, out.data(), bytes, path);
    }

    void IO::read_elements(Tensor& t, std::FILE* f, const std::string& path, bool fortran)
    {
        const size_t bpe = element_bytes(t.dtype);
        const size_t bytes = static_cast<size_t>(t.num_elements) * bpe;
        if (bytes == 0) return;
        const bool device = t.storage->strategy == SushiRuntime::Memory::AllocStrategy::DEVICE;
        if (file_order_matches(t, fortran))
        {
            if (!device)
            {
                read_all(f, t.data(), bytes, path);
                return;
            }
            // file -> pinned chunk i while chunk i-1 is copied to HBM
            hipStream_t s = engine_.get_context().get_queue().native();
            const size_t chunk = std::min(kChunk, bytes);
            Pinned buf0(chunk), buf1(chunk);
            char* bufs[2] = {buf0.bytes(), buf1.bytes()};
            hipEvent_t done[2] = {nullptr, nullptr};
            hip_check(hipEventCreateWithFlags(&done[0], hipEventDisableTiming), "hipEventCreate");
            hip_check(hipEventCreateWithFlags(&done[1], hipEventDisableTiming), "hipEventCreate");
            struct Events
            {
                hipEvent_t* e;
                ~Events()
                {
                    (void)hipEventDestroy(e[0]);
                    (void)hipEventDestroy(e[1]);
                }
            } events{done};
            StreamDrain drain{s};
            char* dst = static_cast<char*>(t.data());
            const size_t n_chunks = (bytes + chunk - 1) / chunk;
            for (size_t i = 0; i < n_chunks; ++i)
            {
                const int b = static_cast<int>(i & 1);
                if (i >= 2) hip_check(hipEventSynchronize(done[b]), "hipEventSynchronize");
                const size_t off = i * chunk, n = std::min(chunk, bytes - off);
                read_all(f, bufs[b], n, path);
                hip_check(hipMemcpyAsync(dst + off, bufs[b], n, hipMemcpyHostToDevice, s),
                          "hipMemcpyAsync(H2D)");
                hip_check(hipEventRecord(done[b], s), "hipEventRecord");
            }
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
            return;
        }
        // general view or other element order: scatter into a host copy of the span
        std::vector<char> in(bytes);
        read_all(f, in.data(), bytes, path);
        const size_t span = static_cast<size_t>(span_elements(t)) * bpe;
        std::vector<char> host;
        char* base;
        if (device)
        {
            host.resize(span);
            hip_check(hipMemcpy(host.data(), t.data(), span, hipMemcpyDeviceToHost), "hipMemcpy(D2H)");
            base = host.data();
        }
        else
        {
            base = static_cast<char*>(t.data());
        }
        for_each_offset(t, fortran, [&](int64_t e, int64_t off) {
            std::memcpy(base + off * bpe, in.data() + e * bpe, bpe);
        });
        if (device)
            hip_check(hipMemcpy(t.data(), host.data(), span, hipMemcpyHostToDevice), "hipMemcpy(H2D)");
    }

    void IO::save_npy(const Tensor& t, const std::string& path)
    {
        SB_THROW_IF(!t.storage && t.num_elements > 0, "save_npy: tensor has no storage");
        engine_.execute().wait();
        File file(path, "wb");
        SB_THROW_IF(!file.f, "Failed to open file: {}", path);
        const std::string pre = npy_header(t.dtype, t.layout, t.shape.data(), t.rank);
        write_all(file.f, pre.data(), pre.size(), path);
        write_elements(t, file.f, path, t.layout == Core::Layout::COLUMN_MAJOR);
        SB_THROW_IF(std::fflush(file.f) != 0, "Failed to write {}", path);
    }

    void IO::load_npy(Tensor& t, const std::string& path)
    {
        File file(path, "rb");
        SB_THROW_IF(!file.f, "Failed to open file for reading: {}", path);
        std::string pre(12, '\0');
        const size_t got = std::fread(&pre[0], 1, 12, file.f);
        pre.resize(got);
        SB_THROW_IF(got < 10 || pre.compare(0, 6, std::string("\x93NUMPY", 6)) != 0,
                    "Invalid .npy file magic.");
        const unsigned major = static_cast<unsigned char>(pre[6]);
        size_t total;
        if (major == 1)
            total = 10 + (static_cast<unsigned char>(pre[8]) |
                          (size_t(static_cast<unsigned char>(pre[9])) << 8));
        else
        {
            SB_THROW_IF((major != 2 && major != 3) || got < 12, "Unsupported .npy format version {}",
                        major);
            size_t hl = 0;
            for (int i = 0; i < 4; ++i) hl |= size_t(static_cast<unsigned char>(pre[8 + i])) << (8 * i);
            total = 12 + hl;
        }
        SB_THROW_IF(total > (size_t(1) << 24), "npy header of {} bytes is not plausible", total);
        if (total > got)
        {
            pre.resize(total);
            read_all(file.f, &pre[got], total - got, path);
        }
        const NpyHeader h = parse_npy_header(pre);
        SB_THROW_IF(h.descr != npy_descr(t.dtype) &&
                        !(h.descr.size() > 1 && h.descr[0] == '=' &&
                          h.descr.substr(1) == std::string(npy_descr(t.dtype)).substr(1)),
                    "npy dtype '{}' does not match the tensor's '{}'", h.descr, npy_descr(t.dtype));
        SB_THROW_IF(static_cast<int>(h.shape.size()) != t.rank,
                    "npy rank {} does not match the tensor's rank {}", h.shape.size(), t.rank);
        for (int i = 0; i < t.rank; ++i)
            SB_THROW_IF(h.shape[i] != t.shape[i], "Shape dimension {} mismatch in .npy header.", i);
        SB_THROW_IF(!t.storage && t.num_elements > 0, "load_npy: tensor has no storage");
        SB_THROW_IF(std::fseek(file.f, static_cast<long>(h.data_offset), SEEK_SET) != 0,
                    "Failed to seek in {}", path);
        read_elements(t, file.f, path, h.fortran_order);
    }

    void IO::save_bin(const Tensor& t, const std::string& path)
    {
        SB_THROW_IF(!t.storage && t.num_elements > 0, "save_bin: tensor has no storage");
        engine_.execute().wait();
        File file(path, "wb");
        SB_THROW_IF(!file.f, "Failed to open file: {}", path);
        write_elements(t, file.f, path, t.layout == Core::Layout::COLUMN_MAJOR);
        SB_THROW_IF(std::fflush(file.f) != 0, "Failed to write {}", path);
    }

    void IO::load_bin(Tensor& t, const std::string& path)
    {
        SB_THROW_IF(!t.storage && t.num_elements > 0, "load_bin: tensor has no storage");
        File file(path, "rb");
        SB_THROW_IF(!file.f, "Failed to open file: {}", path);
        read_elements(t, file.f, path, t.layout == Core::Layout::COLUMN_MAJOR);
    }
} // namespace SushiBLAS

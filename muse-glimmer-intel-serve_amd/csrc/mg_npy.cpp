// .npy I/O between files and device tensors: the reference's fixture and dump
// format (oracle::Tensor's save_npy / load_npy / save_npy_i64,
// src/tensor.h:11-48, src/tensor.cpp:13-224), the files its --dump-hidden and
// --trace-dir write (src/main.cpp:55-76).
//
// Reading: .npy version 1 (16-bit header length) or 2/3 (32-bit), C order,
// descr '<f8', '<f4', '<i8', '<i4' or '|u1'; every value is widened to f64 as
// load_npy does (u1 values stay 0..255), then stored at the requested dtype
// with the twin's rounding (prec::round_act, src/rounding.hpp:64-166: f64 ->
// f32 RNE -> bf16 / f16 RNE, NaN -> 0x7FC0 for bf16 and sign | 0x7E00 for f16).
// Writing: '<f8' tensors and 1-d '<i8' vectors, the header dict padded with
// spaces so that magic + version + length field + dict + '\n' is a multiple of
// 64 bytes, version 1 — the bytes save_npy and save_npy_i64 write.
// Host code: file I/O and conversions on the host, one device copy on the
// context's stream, waited for; nothing is allocated on the device.
#include "mg_internal.hpp"
#include "mg_prims.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace mg
{
    namespace
    {
        struct File
        {
            std::FILE *f = nullptr;
            explicit File(const char *path, const char *mode) : f(std::fopen(path, mode)) {}
            ~File()
            {
                if (f) std::fclose(f);
            }
        };

        struct Header
        {
            std::string descr;
            std::vector<int64_t> shape;
            int64_t count() const
            {
                int64_t n = 1;
                for (int64_t d : shape) n *= d;
                return n;
            }
        };

        // the value text after 'key': in a header dict
        std::string field(const std::string &h, const char *key, const std::string &path)
        {
            const std::string k = std::string("'") + key + "'";
            const size_t at = h.find(k);
            need(at != std::string::npos, "npy: no '" + std::string(key) + "' in the header of " + path);
            size_t i = h.find(':', at + k.size());
            need(i != std::string::npos, "npy: malformed header in " + path);
            ++i;
            while (i < h.size() && h[i] == ' ') ++i;
            return h.substr(i);
        }

        Header read_header(std::FILE *f, const std::string &path)
        {
            unsigned char pre[8];
            need(std::fread(pre, 1, 8, f) == 8 && std::memcmp(pre, "\x93NUMPY", 6) == 0, "npy: not an .npy file: " + path);
            uint32_t hlen = 0;
            if (pre[6] == 1) {
                unsigned char b[2];
                need(std::fread(b, 1, 2, f) == 2, "npy: truncated header in " + path);
                hlen = uint32_t(b[0]) | uint32_t(b[1]) << 8;
            } else {
                unsigned char b[4];
                need(std::fread(b, 1, 4, f) == 4, "npy: truncated header in " + path);
                hlen = uint32_t(b[0]) | uint32_t(b[1]) << 8 | uint32_t(b[2]) << 16 | uint32_t(b[3]) << 24;
            }
            need(hlen < (1u << 24), "npy: header too long in " + path);
            std::string h(hlen, '\0');
            need(std::fread(&h[0], 1, hlen, f) == hlen, "npy: truncated header in " + path);
            Header hd;
            const std::string d = field(h, "descr", path);
            need(d.size() > 2 && d[0] == '\'', "npy: malformed descr in " + path);
            hd.descr = d.substr(1, d.find('\'', 1) - 1);
            need(field(h, "fortran_order", path).rfind("False", 0) == 0, "npy: Fortran order is not supported: " + path);
            const std::string s = field(h, "shape", path);
            const size_t open = s.find('('), close = s.find(')');
            need(open != std::string::npos && close != std::string::npos && close > open,
                 "npy: malformed shape in " + path);
            int64_t cur = -1;
            for (size_t i = open + 1; i < close; ++i) {
                const char c = s[i];
                if (c >= '0' && c <= '9') {
                    cur = (cur < 0 ? 0 : cur) * 10 + (c - '0');
                    need(cur < (int64_t(1) << 40), "npy: dimension too large in " + path);
                } else if (cur >= 0) {
                    hd.shape.push_back(cur);
                    cur = -1;
                }
            }
            if (cur >= 0) hd.shape.push_back(cur);
            return hd;
        }

        // the twin's storage rounding of an f64 value
        uint16_t bf16_bits_of(double v)
        {
            const float f = float(v);
            uint32_t u;
            std::memcpy(&u, &f, 4);
            if (std::isnan(f)) return 0x7fc0;
            return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        }
        uint16_t f16_bits_of(double v)
        {
            const float f = float(v);
            uint32_t u;
            std::memcpy(&u, &f, 4);
            const uint16_t sign = uint16_t((u >> 16) & 0x8000u);
            if (std::isnan(f)) return uint16_t(sign | 0x7e00u);
            const _Float16 h = static_cast<_Float16>(f); // IEEE RNE, subnormals, overflow to inf
            uint16_t b;
            std::memcpy(&b, &h, 2);
            return b;
        }
        double f64_of_bf16(uint16_t b)
        {
            const uint32_t u = uint32_t(b) << 16;
            float f;
            std::memcpy(&f, &u, 4);
            return double(f);
        }
        double f64_of_f16(uint16_t b)
        {
            _Float16 h;
            std::memcpy(&h, &b, 2);
            return double(float(h));
        }
        size_t elem_bytes(int dt)
        {
            return dt == MG_F64 ? 8 : dt == MG_F32 ? 4 : 2;
        }

        void write_header(std::FILE *f, const char *descr, const int64_t *shape, int ndim, const std::string &path)
        {
            std::string d = std::string("{'descr': '") + descr + "', 'fortran_order': False, 'shape': (";
            for (int i = 0; i < ndim; ++i) {
                d += std::to_string(shape[i]);
                if (ndim == 1 || i + 1 < ndim) d += ",";
                if (i + 1 < ndim) d += " ";
            }
            d += "), }";
            const size_t used = 10 + d.size() + 1;
            d.append((64 - used % 64) % 64, ' ');
            d += '\n';
            need(d.size() < 65536, "npy: header too long for " + path);
            const unsigned char pre[10] = {0x93, 'N', 'U', 'M', 'P', 'Y', 1, 0, uint8_t(d.size() & 0xff),
                                           uint8_t(d.size() >> 8)};
            need(std::fwrite(pre, 1, 10, f) == 10 && std::fwrite(d.data(), 1, d.size(), f) == d.size(),
                 "npy: short write: " + path);
        }
    } // namespace

    void npy_info(const char *path, char *descr, int64_t *shape, int max_ndim, int *ndim)
    {
        need(path && ndim, "npy_info: NULL argument");
        File fl(path, "rb");
        need(fl.f != nullptr, std::string("npy: cannot open ") + path);
        const Header h = read_header(fl.f, path);
        need(int(h.shape.size()) <= max_ndim, std::string("npy: more dimensions than the shape buffer holds: ") + path);
        *ndim = int(h.shape.size());
        for (size_t i = 0; i < h.shape.size(); ++i)
            if (shape) shape[i] = h.shape[i];
        if (descr) {
            std::strncpy(descr, h.descr.c_str(), 15);
            descr[15] = '\0';
        }
    }

    void npy_load(mg_ctx *c, const char *path, void *dst, int64_t n, int dt)
    {
        need(path != nullptr, "npy_load: NULL path");
        need(dt == MG_F64 || dt == MG_F32 || dt == MG_BF16 || dt == MG_F16, "npy_load: dtype must be f64, f32, bf16 or f16");
        File fl(path, "rb");
        need(fl.f != nullptr, std::string("npy: cannot open ") + path);
        const Header h = read_header(fl.f, path);
        const int64_t cnt = h.count();
        need(cnt == n, "npy_load: " + std::string(path) + " holds " + std::to_string(cnt) + " values, " +
                           std::to_string(n) + " expected");
        if (n == 0) return;
        need(dst != nullptr, "npy_load: NULL destination");
        // widened to f64, as load_npy reads every descr
        std::vector<double> v(static_cast<size_t>(n));
        bool ok = true;
        auto widen = [&](auto tag) {
            using T = decltype(tag);
            std::vector<T> raw(static_cast<size_t>(n));
            ok = std::fread(raw.data(), sizeof(T), size_t(n), fl.f) == size_t(n);
            for (int64_t i = 0; i < n; ++i) v[size_t(i)] = double(raw[size_t(i)]);
        };
        if (h.descr == "<f8")
            ok = std::fread(v.data(), 8, size_t(n), fl.f) == size_t(n);
        else if (h.descr == "<f4")
            widen(float{});
        else if (h.descr == "<i8")
            widen(int64_t{});
        else if (h.descr == "<i4")
            widen(int32_t{});
        else if (h.descr == "|u1")
            widen(uint8_t{});
        else
            fail("npy: unsupported descr " + h.descr + " in " + path);
        need(ok, std::string("npy: short read: ") + path);
        // stored at the requested dtype with the twin's rounding
        std::vector<unsigned char> out(size_t(n) * elem_bytes(dt));
        for (int64_t i = 0; i < n; ++i) {
            const double x = v[size_t(i)];
            unsigned char *p = out.data() + size_t(i) * elem_bytes(dt);
            if (dt == MG_F64) {
                std::memcpy(p, &x, 8);
            } else if (dt == MG_F32) {
                const float f = float(x);
                std::memcpy(p, &f, 4);
            } else {
                const uint16_t b = dt == MG_BF16 ? bf16_bits_of(x) : f16_bits_of(x);
                std::memcpy(p, &b, 2);
            }
        }
        check(hipMemcpyAsync(dst, out.data(), out.size(), hipMemcpyHostToDevice, c->stream), "npy_load: copy");
        check(hipStreamSynchronize(c->stream), "npy_load: wait");
    }

    void npy_save(mg_ctx *c, const char *path, const void *src, int dt, const int64_t *shape, int ndim)
    {
        need(path != nullptr, "npy_save: NULL path");
        need(dt == MG_F64 || dt == MG_F32 || dt == MG_BF16 || dt == MG_F16, "npy_save: dtype must be f64, f32, bf16 or f16");
        need(ndim >= 0 && ndim <= 32 && (ndim == 0 || shape), "npy_save: bad shape");
        int64_t n = 1;
        for (int i = 0; i < ndim; ++i) {
            need(shape[i] >= 0, "npy_save: negative dimension");
            n *= shape[i];
        }
        std::vector<unsigned char> raw(size_t(n) * elem_bytes(dt));
        if (n > 0) {
            need(src != nullptr, "npy_save: NULL source");
            check(hipMemcpyAsync(raw.data(), src, raw.size(), hipMemcpyDeviceToHost, c->stream), "npy_save: copy");
            check(hipStreamSynchronize(c->stream), "npy_save: wait");
        }
        // save_npy writes f64: every storage value widens exactly
        std::vector<double> v(static_cast<size_t>(n));
        for (int64_t i = 0; i < n; ++i) {
            const unsigned char *p = raw.data() + size_t(i) * elem_bytes(dt);
            if (dt == MG_F64) {
                std::memcpy(&v[size_t(i)], p, 8);
            } else if (dt == MG_F32) {
                float f;
                std::memcpy(&f, p, 4);
                v[size_t(i)] = double(f);
            } else {
                uint16_t b;
                std::memcpy(&b, p, 2);
                v[size_t(i)] = dt == MG_BF16 ? f64_of_bf16(b) : f64_of_f16(b);
            }
        }
        File fl(path, "wb");
        need(fl.f != nullptr, std::string("npy: cannot write ") + path);
        write_header(fl.f, "<f8", shape, ndim, path);
        need(std::fwrite(v.data(), 8, size_t(n), fl.f) == size_t(n), std::string("npy: short write: ") + path);
    }

    void npy_save_i64(mg_ctx *c, const char *path, const int64_t *src, int64_t n)
    {
        need(path != nullptr && n >= 0, "npy_save_i64: bad arguments");
        std::vector<int64_t> v(static_cast<size_t>(n));
        if (n > 0) {
            need(src != nullptr, "npy_save_i64: NULL source");
            check(hipMemcpyAsync(v.data(), src, size_t(n) * 8, hipMemcpyDeviceToHost, c->stream), "npy_save_i64: copy");
            check(hipStreamSynchronize(c->stream), "npy_save_i64: wait");
        }
        File fl(path, "wb");
        need(fl.f != nullptr, std::string("npy: cannot write ") + path);
        const int64_t shape[1] = {n};
        write_header(fl.f, "<i8", shape, 1, path);
        need(std::fwrite(v.data(), 8, size_t(n), fl.f) == size_t(n), std::string("npy: short write: ") + path);
    }
} // namespace mg

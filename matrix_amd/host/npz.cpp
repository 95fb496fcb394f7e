// npz.cpp -- matrix::save_as_npz and matrix::load_npz: the on-disk boundary of the graph layer.
//
// save_as_npz writes what the reference's save_as_npz writes (Matrix.mm:3748-4085, declared
// matrix.h:1237), byte for byte: one uncompressed .npy per matrix, named arr_<i>.npy, inside a
// ZIP archive with STORED entries.
//   - .npy: magic "\x93NUMPY", version 1.0, a little-endian u16 header length, then the header
//     {'descr': '<f4', 'fortran_order': False, 'shape': (3,4), } (the shape's items joined by ","
//     with no space, a 1-tuple as "(5,)", rank 0 as "()") padded with spaces and a final '\n' so
//     that 10 + its length is a multiple of 64, then the row-major element bytes.
//   - descr per dtype: <f4 <f2 <i4 <u4 <i2 <u2 |u1 |b1 |i1 <i8 <u8 <c8; BFloat16 has no numpy
//     dtype and is rejected.
//   - ZIP: per entry a local header (version 20, no flags, method 0, zero time and date, the
//     CRC-32 and size twice, the name, no extra field) and the .npy bytes; then one central
//     directory record per entry (made by / needed 20, the local header's offset) and the end
//     record.  No ZIP64: more than 65535 entries, an entry over 4 GiB or a file over 4 GiB is
//     rejected before the file is opened.
// Values come from the device when a matrix was computed there (a strided view is made
// contiguous on the device first, as the reference's astype(type, true) does).
//
// load_npz has no counterpart in the reference: it reads such archives back (and numpy's own
// np.savez files, whose local headers carry ZIP64 size fields) into host leaves, uploaded on
// the next compile.  Entries must be STORED; their CRC-32 is checked.
#include "matrix.hpp"

#include <array>
#include <cstdio>
#include <fstream>

namespace {

// ------------------------------------------------------------------ CRC-32 (ISO-HDLC / ZIP)
// Reflected polynomial 0xEDB88320, initial value and final xor 0xFFFFFFFF; a 256-entry table of
// the byte-at-a-time division.
const std::array<uint32_t, 256>& crc_table() {
    static const std::array<uint32_t, 256> t = [] {
        std::array<uint32_t, 256> r{};
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t c = i;
            for (int k = 0; k < 8; k++) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            r[i] = c;
        }
        return r;
    }();
    return t;
}

uint32_t crc32(const uint8_t* p, size_t n) {
    const auto& t = crc_table();
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; i++) c = t[(c ^ p[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

// ------------------------------------------------------------------ little-endian fields
void put_le(std::vector<uint8_t>& out, uint64_t v, int bytes) {
    for (int i = 0; i < bytes; i++) out.push_back((uint8_t)(v >> (8 * i)));
}

uint64_t get_le(const uint8_t* p, int bytes) {
    uint64_t v = 0;
    for (int i = bytes - 1; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

// ------------------------------------------------------------------ .npy
const char* npy_descr(dtype t) {
    switch (t) {
    case dtype::Float: return "<f4";
    case dtype::Float16: return "<f2";
    case dtype::Int32: return "<i4";
    case dtype::UInt32: return "<u4";
    case dtype::Int16: return "<i2";
    case dtype::UInt16: return "<u2";
    case dtype::UInt8: return "|u1";
    case dtype::Bool: return "|b1";
    case dtype::Int8: return "|i1";
    case dtype::Int64: return "<i8";
    case dtype::UInt64: return "<u8";
    case dtype::Complex64: return "<c8";
    case dtype::BFloat16: break;
    }
    throw std::runtime_error(std::string("save_as_npz: ") + dtype_name(t) + " has no numpy dtype");
}

std::string npy_header(const matrix& m) {
    std::string shape = "(";
    for (uint32_t i = 0; i < m.dims; i++) {
        shape += std::to_string(m.shape()[i]);
        if (m.dims == 1 || i + 1 < m.dims) shape += ",";
    }
    shape += ")";
    std::string h = std::string("{'descr': '") + npy_descr(m.type) + "', 'fortran_order': False, 'shape': " + shape + ", }";
    const size_t used = 10 + h.size() + 1;                   // magic, version, length, header, '\n'
    h.append((64 - used % 64) % 64, ' ');
    h.push_back('\n');
    return h;
}

// The npy file of one matrix: header, then its elements in row-major order.
std::vector<uint8_t> npy_file(const matrix& m) {
    const std::string h = npy_header(m);
    std::vector<uint8_t> out = {0x93, 'N', 'U', 'M', 'P', 'Y', 1, 0};
    put_le(out, h.size(), 2);
    out.insert(out.end(), h.begin(), h.end());
    matrix src = m;
    // a view computed on the device is packed there (one strided copy), then read back whole
    if (!m.is_contiguous() && !m.storage->host_is_source) {
        src = m.astype(m.type, true);
        src.eval();
    }
    const std::vector<uint8_t> data = src.to_host_bytes();
    out.insert(out.end(), data.begin(), data.end());
    return out;
}

// ------------------------------------------------------------------ .npy header parsing
struct NpyHeader {
    dtype type = dtype::Float;
    bool fortran = false;
    std::vector<size_m> shape;
};

[[noreturn]] void bad_npy(const std::string& name, const std::string& why) {
    throw std::runtime_error("load_npz: " + name + ": " + why);
}

dtype dtype_of_descr(const std::string& d, const std::string& name) {
    static const std::pair<const char*, dtype> table[] = {
        {"<f4", dtype::Float}, {"<f2", dtype::Float16}, {"<i4", dtype::Int32}, {"<u4", dtype::UInt32},
        {"<i2", dtype::Int16}, {"<u2", dtype::UInt16}, {"|u1", dtype::UInt8}, {"<u1", dtype::UInt8},
        {"|b1", dtype::Bool},  {"<b1", dtype::Bool},   {"|i1", dtype::Int8},  {"<i1", dtype::Int8},
        {"<i8", dtype::Int64}, {"<u8", dtype::UInt64}, {"<c8", dtype::Complex64}};
    for (const auto& e : table)
        if (d == e.first) return e.second;
    bad_npy(name, "unsupported descr '" + d + "'");
}

// The value after 'key': in a numpy header dict (a Python literal written by numpy or by
// save_as_npz), as raw text up to the matching delimiter.
std::string dict_value(const std::string& h, const std::string& key, const std::string& name) {
    const std::string k = "'" + key + "'";
    size_t p = h.find(k);
    if (p == std::string::npos) bad_npy(name, "header has no " + k);
    p = h.find(':', p + k.size());
    if (p == std::string::npos) bad_npy(name, "header entry " + k + " has no value");
    p++;
    while (p < h.size() && h[p] == ' ') p++;
    if (p >= h.size()) bad_npy(name, "header entry " + k + " has no value");
    size_t e;
    if (h[p] == '\'') {
        e = h.find('\'', p + 1);
        if (e == std::string::npos) bad_npy(name, "unterminated string in header");
        return h.substr(p + 1, e - p - 1);
    }
    if (h[p] == '(') {
        e = h.find(')', p);
        if (e == std::string::npos) bad_npy(name, "unterminated shape tuple in header");
        return h.substr(p, e - p + 1);
    }
    e = h.find_first_of(",}", p);
    if (e == std::string::npos) bad_npy(name, "malformed header");
    return h.substr(p, e - p);
}

NpyHeader parse_npy(const uint8_t* p, size_t n, size_t* data_off, const std::string& name) {
    static const uint8_t magic[6] = {0x93, 'N', 'U', 'M', 'P', 'Y'};
    if (n < 10 || std::memcmp(p, magic, 6) != 0) bad_npy(name, "not an .npy file");
    const int major = p[6];
    size_t hl, ho;
    if (major == 1) { hl = get_le(p + 8, 2); ho = 10; }
    else if (major == 2 || major == 3) {
        if (n < 12) bad_npy(name, "truncated header");
        hl = get_le(p + 8, 4); ho = 12;
    } else bad_npy(name, "npy version " + std::to_string(major) + " is not 1, 2 or 3");
    if (ho + hl > n) bad_npy(name, "truncated header");
    const std::string h(reinterpret_cast<const char*>(p + ho), hl);
    NpyHeader r;
    r.type = dtype_of_descr(dict_value(h, "descr", name), name);
    const std::string fo = dict_value(h, "fortran_order", name);
    if (fo == "True") r.fortran = true;
    else if (fo != "False") bad_npy(name, "fortran_order is neither True nor False");
    const std::string sh = dict_value(h, "shape", name);
    size_t i = 1;
    while (i < sh.size()) {
        while (i < sh.size() && (sh[i] == ' ' || sh[i] == ',')) i++;
        if (i >= sh.size() || sh[i] == ')') break;
        size_t j = i;
        uint64_t v = 0;
        while (j < sh.size() && sh[j] >= '0' && sh[j] <= '9') {
            v = v * 10 + (uint64_t)(sh[j] - '0');
            if (v > 0xFFFFFFFFull) bad_npy(name, "an extent does not fit 32 bits");
            j++;
        }
        if (j == i) bad_npy(name, "malformed shape " + sh);
        r.shape.push_back((size_m)v);
        i = j;
    }
    *data_off = ho + hl;
    return r;
}

}  // namespace

// ------------------------------------------------------------------ writer
void matrix::save_as_npz(std::vector<matrix> input, std::string file_path) {
    constexpr uint64_t kMaxEntries = 0xFFFF, kMax32 = 0xFFFFFFFFull;
    if (input.size() > kMaxEntries)
        throw std::runtime_error("save_as_npz: " + std::to_string(input.size()) +
                                 " arrays exceed the 65535 entries of a ZIP without ZIP64");
    std::vector<std::pair<std::string, std::vector<uint8_t>>> entries;
    entries.reserve(input.size());
    for (size_t i = 0; i < input.size(); i++) {
        const matrix& m = input[i];
        if (!m.storage) throw std::invalid_argument("save_as_npz: arr_" + std::to_string(i) + " is empty");
        npy_descr(m.type);                                  // reject BFloat16 before any work
        const uint64_t data_bytes = (uint64_t)m.total_size() * dtype_size(m.type);
        if (data_bytes > kMax32)
            throw std::runtime_error("save_as_npz: arr_" + std::to_string(i) + " holds " + std::to_string(data_bytes) +
                                     " bytes, over the 4 GiB of a ZIP entry without ZIP64");
        entries.emplace_back("arr_" + std::to_string(i) + ".npy", npy_file(m));
        if (entries.back().second.size() > kMax32)
            throw std::runtime_error("save_as_npz: arr_" + std::to_string(i) + " is " +
                                     std::to_string(entries.back().second.size()) +
                                     " bytes as .npy, over the 4 GiB of a ZIP entry without ZIP64");
    }
    uint64_t file_bytes = 22;
    for (const auto& e : entries) file_bytes += 30 + 46 + 2 * e.first.size() + e.second.size();
    if (file_bytes > kMax32)
        throw std::runtime_error("save_as_npz: the archive would be " + std::to_string(file_bytes) +
                                 " bytes, over the 4 GiB of a ZIP without ZIP64");

    std::vector<uint8_t> central;
    std::ofstream f(file_path, std::ios::binary);
    if (!f) throw std::runtime_error("save_as_npz: cannot open " + file_path + " for writing");
    uint64_t pos = 0;
    auto emit = [&](const std::vector<uint8_t>& b) {
        f.write(reinterpret_cast<const char*>(b.data()), (std::streamsize)b.size());
        pos += b.size();
    };
    for (const auto& [name, blob] : entries) {
        const uint32_t crc = crc32(blob.data(), blob.size());
        const uint64_t local = pos;
        std::vector<uint8_t> h;
        put_le(h, 0x04034b50u, 4);
        put_le(h, 20, 2);                  // version needed
        put_le(h, 0, 2);                   // flags
        put_le(h, 0, 2);                   // method: stored
        put_le(h, 0, 2);                   // time
        put_le(h, 0, 2);                   // date
        put_le(h, crc, 4);
        put_le(h, blob.size(), 4);         // compressed size
        put_le(h, blob.size(), 4);         // uncompressed size
        put_le(h, name.size(), 2);
        put_le(h, 0, 2);                   // extra length
        h.insert(h.end(), name.begin(), name.end());
        emit(h);
        emit(blob);

        put_le(central, 0x02014b50u, 4);
        put_le(central, 20, 2);            // version made by
        put_le(central, 20, 2);            // version needed
        put_le(central, 0, 2);             // flags
        put_le(central, 0, 2);             // method
        put_le(central, 0, 2);             // time
        put_le(central, 0, 2);             // date
        put_le(central, crc, 4);
        put_le(central, blob.size(), 4);
        put_le(central, blob.size(), 4);
        put_le(central, name.size(), 2);
        put_le(central, 0, 2);             // extra length
        put_le(central, 0, 2);             // comment length
        put_le(central, 0, 2);             // disk
        put_le(central, 0, 2);             // internal attributes
        put_le(central, 0, 4);             // external attributes
        put_le(central, local, 4);
        central.insert(central.end(), name.begin(), name.end());
    }
    const uint64_t cd_off = pos;
    emit(central);
    std::vector<uint8_t> end;
    put_le(end, 0x06054b50u, 4);
    put_le(end, 0, 2);                     // this disk
    put_le(end, 0, 2);                     // disk of the central directory
    put_le(end, entries.size(), 2);
    put_le(end, entries.size(), 2);
    put_le(end, central.size(), 4);
    put_le(end, cd_off, 4);
    put_le(end, 0, 2);                     // comment length
    emit(end);
    if (!f) throw std::runtime_error("save_as_npz: writing " + file_path + " failed");
}

// ------------------------------------------------------------------ loader
std::vector<matrix> matrix::load_npz(const std::string& file_path, std::vector<std::string>* names) {
    std::ifstream f(file_path, std::ios::binary);
    if (!f) throw std::runtime_error("load_npz: cannot open " + file_path);
    std::vector<uint8_t> z((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    const size_t n = z.size();
    auto need = [&](uint64_t off, uint64_t len, const char* what) {
        if (off > n || len > n - off) throw std::runtime_error(std::string("load_npz: truncated archive (") + what + ")");
    };
    // end of central directory: the last signature within the final 64 KiB + 22 bytes
    if (n < 22) throw std::runtime_error("load_npz: " + file_path + " is not a ZIP archive");
    size_t eocd = std::string::npos;
    const size_t lo = n > 65557 ? n - 65557 : 0;
    for (size_t p = n - 22 + 1; p-- > lo;)
        if (get_le(&z[p], 4) == 0x06054b50u) { eocd = p; break; }
    if (eocd == std::string::npos) throw std::runtime_error("load_npz: " + file_path + " has no ZIP end record");
    uint64_t count = get_le(&z[eocd + 10], 2);
    uint64_t cd_size = get_le(&z[eocd + 12], 4);
    uint64_t cd_off = get_le(&z[eocd + 16], 4);
    if (count == 0xFFFF || cd_size == 0xFFFFFFFFull || cd_off == 0xFFFFFFFFull) {
        // ZIP64: locator just before the end record, pointing at the ZIP64 end record
        if (eocd < 20 || get_le(&z[eocd - 20], 4) != 0x07064b50u)
            throw std::runtime_error("load_npz: ZIP64 archive without a ZIP64 locator");
        const uint64_t z64 = get_le(&z[eocd - 20 + 8], 8);
        need(z64, 56, "ZIP64 end record");
        if (get_le(&z[z64], 4) != 0x06064b50u) throw std::runtime_error("load_npz: bad ZIP64 end record");
        count = get_le(&z[z64 + 32], 8);
        cd_size = get_le(&z[z64 + 40], 8);
        cd_off = get_le(&z[z64 + 48], 8);
    }
    need(cd_off, cd_size, "central directory");
    std::vector<matrix> out;
    if (names) names->clear();
    uint64_t p = cd_off;
    for (uint64_t e = 0; e < count; e++) {
        need(p, 46, "central directory record");
        if (get_le(&z[p], 4) != 0x02014b50u) throw std::runtime_error("load_npz: bad central directory record");
        const uint64_t method = get_le(&z[p + 10], 2);
        const uint32_t crc = (uint32_t)get_le(&z[p + 16], 4);
        uint64_t csize = get_le(&z[p + 20], 4), usize = get_le(&z[p + 24], 4);
        const uint64_t nl = get_le(&z[p + 28], 2), xl = get_le(&z[p + 30], 2), cl = get_le(&z[p + 32], 2);
        uint64_t local = get_le(&z[p + 42], 4);
        need(p + 46, nl + xl + cl, "central directory record");
        std::string name(reinterpret_cast<const char*>(&z[p + 46]), nl);
        // ZIP64 extra field (id 1): the 64-bit values of the fields that read 0xFFFFFFFF, in order
        for (uint64_t q = p + 46 + nl; q + 4 <= p + 46 + nl + xl;) {
            const uint64_t id = get_le(&z[q], 2), len = get_le(&z[q + 2], 2);
            if (q + 4 + len > p + 46 + nl + xl) break;
            if (id == 1) {
                uint64_t r = q + 4;
                auto take = [&](uint64_t& v) {
                    if (v == 0xFFFFFFFFull && r + 8 <= q + 4 + len) { v = get_le(&z[r], 8); r += 8; }
                };
                take(usize);
                take(csize);
                take(local);
            }
            q += 4 + len;
        }
        p += 46 + nl + xl + cl;
        if (method != 0)
            throw std::runtime_error("load_npz: entry " + name + " is compressed (method " + std::to_string(method) +
                                     "); only stored entries are read");
        if (csize != usize) throw std::runtime_error("load_npz: entry " + name + " has differing sizes");
        need(local, 30, "local header");
        if (get_le(&z[local], 4) != 0x04034b50u) throw std::runtime_error("load_npz: bad local header for " + name);
        const uint64_t data = local + 30 + get_le(&z[local + 26], 2) + get_le(&z[local + 28], 2);
        need(data, csize, "entry data");
        if (crc32(&z[data], csize) != crc) throw std::runtime_error("load_npz: CRC-32 mismatch in " + name);
        size_t doff = 0;
        const NpyHeader h = parse_npy(&z[data], csize, &doff, name);
        uint64_t count_el = 1;
        for (size_m s : h.shape) count_el *= s;
        if (csize - doff != count_el * dtype_size(h.type))
            bad_npy(name, "holds " + std::to_string(csize - doff) + " data bytes, the header asks for " +
                              std::to_string(count_el * dtype_size(h.type)));
        matrix m;
        if (!h.fortran) {
            m = from_bytes(h.shape, h.type, &z[data + doff]);
        } else {                                            // column-major: the reversed shape, transposed
            std::vector<size_m> rev(h.shape.rbegin(), h.shape.rend()), order(h.shape.size());
            for (size_t d = 0; d < order.size(); d++) order[d] = (size_m)(order.size() - 1 - d);
            m = from_bytes(rev, h.type, &z[data + doff]).transpose(order);
        }
        out.push_back(m);
        if (names) names->push_back(name.size() > 4 && name.compare(name.size() - 4, 4, ".npy") == 0
                                        ? name.substr(0, name.size() - 4) : name);
    }
    return out;
}

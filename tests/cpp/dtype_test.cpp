// dtype_test.cpp -- result dtypes of the graph's binary ops (promote_types, scalar_operand_type)
// and mixed-dtype graphs on the GPU.
//
//   dtype_test cpu         promote_types against the reference's 13 x 13 table (matrix.h:166-180),
//                          written out below one letter per entry; scalar_operand_type's cases
//                          (matrix.h:1815-1840); the dtype and the casts of the nodes that
//                          operator+ - * / and max / min / equal build; touches no device
//   dtype_test gpu <dir>   mixed-dtype graphs evaluated on the GPU; writes every case's operands
//                          and result as raw bytes into <dir> with a manifest, which the Python
//                          test checks against the oracle in the promoted dtype
//
// Prints "PASS <name>" / "FAIL <name>: <why>" per case; exit status 1 if any case failed.
#include "../../matrix_amd/host/matrix.hpp"

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <limits>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

static int g_fail = 0;

#define EXPECT(cond, msg)                                                     \
    do {                                                                      \
        if (!(cond)) throw std::runtime_error(std::string(msg));              \
    } while (0)

static void run(const char* name, void (*fn)()) {
    try {
        fn();
        std::printf("PASS %s\n", name);
    } catch (const std::exception& e) {
        std::printf("FAIL %s: %s\n", name, e.what());
        g_fail++;
    }
    std::fflush(stdout);
}

static dtype from_letter(char c) {
    switch (c) {
    case 'f': return dtype::Float;
    case 'h': return dtype::Float16;
    case 'B': return dtype::UInt8;
    case 'i': return dtype::Int32;
    case 's': return dtype::Int16;
    case 'I': return dtype::UInt32;
    case 'S': return dtype::UInt16;
    case '?': return dtype::Bool;
    case 'b': return dtype::Int8;
    case 'c': return dtype::Complex64;
    case 'r': return dtype::BFloat16;
    case 'l': return dtype::Int64;
    case 'L': return dtype::UInt64;
    }
    throw std::logic_error(std::string("bad dtype letter ") + c);
}

// type_rules (matrix.h:166-180): row a, column b, both in dtype-code order Float, Float16, UInt8,
// Int32, Int16, UInt32, UInt16, Bool, Int8, Complex64, BFloat16, Int64, UInt64.  Letters:
// f Float, h Float16, B UInt8, i Int32, s Int16, I UInt32, S UInt16, ? Bool, b Int8, c Complex64,
// r BFloat16, l Int64, L UInt64.
static const char* const kTypeRules[13] = {
    "fffffffffcfff",   // Float
    "fhfffffhfcfff",   // Float16
    "ffBisISBscflL",   // UInt8
    "ffiiiiiiicflf",   // Int32
    "ffsisiisscflf",   // Int16
    "ffIiiIIIicflL",   // UInt32
    "ffSiiISSicflL",   // UInt16
    "fhBisIS?bcrlL",   // Bool
    "ffsisiibbcflf",   // Int8
    "ccccccccccccc",   // Complex64
    "fffffffrfcrff",   // BFloat16
    "fflllllllcflf",   // Int64
    "ffLffLLLfcffL",   // UInt64
};

static void promote_types_table() {
    int bad = 0;
    std::string first;
    for (int a = 0; a < 13; a++) {
        EXPECT(std::string(kTypeRules[a]).size() == 13, "table row width");
        for (int b = 0; b < 13; b++) {
            const dtype want = from_letter(kTypeRules[a][b]);
            const dtype got = promote_types((dtype)a, (dtype)b);
            if (got != want) {
                if (!bad) first = std::string(dtype_name((dtype)a)) + " + " + dtype_name((dtype)b) + " -> " +
                                  dtype_name(got) + ", table " + dtype_name(want);
                bad++;
            }
        }
    }
    EXPECT(bad == 0, std::to_string(bad) + " of 169 pairs differ, first: " + first);
}

template <typename T>
static void want_scalar(T v, dtype m, dtype want, const char* what) {
    const dtype got = scalar_operand_type(v, m);
    EXPECT(got == want, std::string(what) + ": got " + dtype_name(got) + ", want " + dtype_name(want));
}

static void scalar_operand_types() {
    // m's own dtype whenever it holds the value
    want_scalar(2, dtype::UInt8, dtype::UInt8, "uint8 * 2");
    want_scalar(0.5f, dtype::Float16, dtype::Float16, "half * 0.5f");
    want_scalar(0.5, dtype::BFloat16, dtype::BFloat16, "bf16 * 0.5");
    want_scalar(1e30, dtype::BFloat16, dtype::BFloat16, "bf16 has Float's range");
    want_scalar(7, dtype::Float, dtype::Float, "float * 7");
    want_scalar(3.0f, dtype::Complex64, dtype::Complex64, "complex * 3.0f");
    want_scalar(true, dtype::Int16, dtype::Int16, "bool scalar adopts m");
    want_scalar(true, dtype::Bool, dtype::Bool, "bool scalar next to bool");
    // a float scalar next to an integer matrix is Float
    want_scalar(0.5f, dtype::Int32, dtype::Float, "int32 + 0.5f");
    want_scalar(2.0, dtype::UInt8, dtype::Float, "uint8 + 2.0");
    want_scalar(1.0f, dtype::Bool, dtype::Float, "bool + 1.0f");
    // Float16's range
    want_scalar(70000.0, dtype::Float16, dtype::Float, "f16 + 70000.0");
    want_scalar(65504.0f, dtype::Float16, dtype::Float16, "f16 + 65504");
    want_scalar(-65504, dtype::Float16, dtype::Float16, "f16 - 65504 (int)");
    want_scalar(70000, dtype::Float16, dtype::Float, "f16 + 70000 (int)");
    want_scalar(std::numeric_limits<float>::quiet_NaN(), dtype::Float16, dtype::Float, "f16 + NaN");
    // integers that do not fit m
    want_scalar(300, dtype::UInt8, dtype::Int32, "uint8 + 300");
    want_scalar(-1, dtype::UInt8, dtype::Int32, "uint8 - 1 (int scalar -1)");
    want_scalar(70000, dtype::Int16, dtype::Int32, "int16 + 70000");
    want_scalar(128, dtype::Int8, dtype::Int32, "int8 + 128");
    want_scalar(1, dtype::Bool, dtype::Int32, "bool + 1");
    want_scalar(3000000000LL, dtype::UInt32, dtype::UInt32, "uint32 + 3e9 fits");
    want_scalar(3000000000LL, dtype::UInt16, dtype::UInt32, "uint16 + 3e9");
    want_scalar(3000000000LL, dtype::Int32, dtype::Int64, "int32 + 3e9");
    want_scalar(5000000000LL, dtype::UInt32, dtype::Int64, "uint32 + 5e9");
    want_scalar(-1, dtype::UInt64, dtype::Int32, "uint64 - 1");
    want_scalar(std::numeric_limits<uint64_t>::max(), dtype::UInt64, dtype::UInt64, "uint64 + UINT64_MAX");
    want_scalar(std::numeric_limits<uint64_t>::max(), dtype::UInt8, dtype::UInt64, "uint8 + UINT64_MAX");
    want_scalar(std::numeric_limits<int64_t>::min(), dtype::Int64, dtype::Int64, "int64 + INT64_MIN");
    bool threw = false;
    try { (void)scalar_operand_type(std::numeric_limits<uint64_t>::max(), dtype::Int64); }
    catch (const std::overflow_error&) { threw = true; }
    EXPECT(threw, "int64 + UINT64_MAX must throw overflow_error");
}

// The dtype operator+ gives, and the cast nodes it inserts (Matrix.mm:8312-8315).
static void graph_result_dtypes() {
    for (int a = 0; a < 13; a++) {
        for (int b = 0; b < 13; b++) {
            if (a == (int)dtype::Complex64 || b == (int)dtype::Complex64) continue;
            matrix x = matrix::leaf({4, 3}, (dtype)a), y = matrix::leaf({3}, (dtype)b);
            const dtype want = from_letter(kTypeRules[a][b]);
            for (matrix r : {x + y, x - y, x * y, x / y, matrix::max(x, y), matrix::min(x, y), matrix::equal(x, y)}) {
                EXPECT(r.type == want, std::string("result of ") + dtype_name((dtype)a) + ", " + dtype_name((dtype)b));
                const matrix& l = r.tape->input_at(0);
                const matrix& rr = r.tape->input_at(1);
                EXPECT(l.type == want && rr.type == want, "operands cast to the promoted dtype");
                EXPECT((a == (int)want) == (l.tape == nullptr), "a cast node only where the dtype changes");
                EXPECT((b == (int)want) == (rr.tape == nullptr), "b cast node only where the dtype changes");
            }
        }
    }
    matrix i32 = matrix::leaf({8}, dtype::Int32), f16 = matrix::leaf({8}, dtype::Float16), u8 = matrix::leaf({8}, dtype::UInt8);
    EXPECT((i32 + 0.5f).type == dtype::Float, "int32 + 0.5f is Float");
    EXPECT((0.5f * i32).type == dtype::Float, "0.5f * int32 is Float");
    EXPECT((f16 + 70000.0).type == dtype::Float, "f16 + 70000.0 is Float");
    EXPECT((f16 * 0.5f).type == dtype::Float16, "f16 * 0.5f stays Float16");
    EXPECT((u8 + 300).type == dtype::Int32, "uint8 + 300 is Int32");
    EXPECT((u8 * 2).type == dtype::UInt8, "uint8 * 2 stays UInt8");
    EXPECT((u8 - 1.0).type == dtype::Float, "uint8 - 1.0 is Float");
    // the scalar's stored value is exact in its own dtype
    matrix s = matrix::scalar(3000000000LL, scalar_operand_type(3000000000LL, dtype::Int32));
    EXPECT(s.type == dtype::Int64 && s.to_host<int64_t>()[0] == 3000000000LL, "int64 scalar stored exactly");
    matrix big = matrix::scalar(std::numeric_limits<uint64_t>::max(), dtype::UInt64);
    EXPECT(big.to_host<uint64_t>()[0] == std::numeric_limits<uint64_t>::max(), "uint64 scalar stored exactly");
}

// ------------------------------------------------------------------ gpu
template <typename T>
static std::vector<T> ints(size_t n, uint64_t seed, int64_t lo, int64_t hi) {
    std::mt19937_64 g(seed);
    std::uniform_int_distribution<int64_t> d(lo, hi);
    std::vector<T> v(n);
    for (auto& x : v) x = (T)d(g);
    return v;
}

static std::vector<uint16_t> halfs(size_t n, uint64_t seed, float scale) {
    std::mt19937_64 g(seed);
    std::normal_distribution<float> d(0.0f, 1.0f);
    std::vector<uint16_t> v(n);
    for (auto& x : v) {
        _Float16 h = (_Float16)(d(g) * scale);
        std::memcpy(&x, &h, 2);
    }
    return v;
}

static std::string g_dir;

static std::string shape_str(const matrix& m) {
    std::string s;
    for (uint32_t i = 0; i < m.dims; i++) s += (i ? "," : "") + std::to_string(m.shape()[i]);
    return s;
}

static void dump(const std::string& name, const matrix& m) {
    const std::vector<uint8_t> b = m.to_host_bytes();
    std::ofstream f(g_dir + "/" + name + ".bin", std::ios::binary);
    f.write(reinterpret_cast<const char*>(b.data()), (std::streamsize)b.size());
}

// One case: r = a op b evaluated on the GPU; the manifest line names op, each operand's dtype code
// and shape, and the result's.
static void emit(std::ofstream& man, const std::string& name, int op, const matrix& a, const matrix& b, matrix r) {
    r.eval();
    dump(name + "_a", a);
    dump(name + "_b", b);
    dump(name + "_r", r);
    man << name << "|" << op << "|" << (int)a.type << "|" << shape_str(a) << "|" << (int)b.type << "|" << shape_str(b)
        << "|" << (int)r.type << "|" << shape_str(r) << "\n";
}

static void gpu_mixed_graphs() {
    std::ofstream man(g_dir + "/manifest.txt");
    EXPECT(man.good(), "cannot write the manifest into " + g_dir);
    const int ADD = 0, SUB = 1, MUL = 2, MAX = 4, EQ = 6;
    {   // i32 + f16 -> Float
        matrix a = matrix::from_host<int32_t>({64, 33}, ints<int32_t>(64 * 33, 1, -1000, 1000));
        matrix b = matrix::from_host<uint16_t>({33}, halfs(33, 2, 10.0f), dtype::Float16);
        emit(man, "i32_add_f16", ADD, a, b, a + b);
    }
    {   // u8 + i8 -> Int16
        matrix a = matrix::from_host<uint8_t>({40, 50}, ints<uint8_t>(40 * 50, 3, 0, 255));
        matrix b = matrix::from_host<int8_t>({50}, ints<int8_t>(50, 4, -128, 127));
        emit(man, "u8_add_i8", ADD, a, b, a + b);
    }
    {   // int32 * 0.5f -> Float (the scalar widens the result instead of truncating to 0)
        matrix a = matrix::from_host<int32_t>({300}, ints<int32_t>(300, 5, -100000, 100000));
        matrix s = matrix::scalar(0.5f, scalar_operand_type(0.5f, a.type));
        emit(man, "i32_mul_half", MUL, a, s, a * s);
    }
    {   // f16 + 70000.0 -> Float
        matrix a = matrix::from_host<uint16_t>({257}, halfs(257, 6, 100.0f), dtype::Float16);
        matrix s = matrix::scalar(70000.0, scalar_operand_type(70000.0, a.type));
        emit(man, "f16_add_70000", ADD, a, s, a + s);
    }
    {   // u8 * 2 -> UInt8 (wraps)
        matrix a = matrix::from_host<uint8_t>({512}, ints<uint8_t>(512, 7, 0, 255));
        matrix s = matrix::scalar(2, scalar_operand_type(2, a.type));
        emit(man, "u8_mul_2", MUL, a, s, a * s);
    }
    {   // u8 + 300 -> Int32
        matrix a = matrix::from_host<uint8_t>({100}, ints<uint8_t>(100, 8, 0, 255));
        matrix s = matrix::scalar(300, scalar_operand_type(300, a.type));
        emit(man, "u8_add_300", ADD, a, s, a + s);
    }
    {   // u32 - i32 -> Int32 (wraps)
        matrix a = matrix::from_host<uint32_t>({16, 16}, ints<uint32_t>(256, 9, 0, 4294967295LL));
        matrix b = matrix::from_host<int32_t>({16, 16}, ints<int32_t>(256, 10, -2147483647LL, 2147483647LL));
        emit(man, "u32_sub_i32", SUB, a, b, a - b);
    }
    {   // i64 + u64 -> Float
        matrix a = matrix::from_host<int64_t>({128}, ints<int64_t>(128, 11, -(1LL << 40), 1LL << 40));
        matrix b = matrix::from_host<uint64_t>({128}, ints<uint64_t>(128, 12, 0, 1LL << 50));
        emit(man, "i64_add_u64", ADD, a, b, a + b);
    }
    {   // max(f16, i32 scalar) -> Float
        matrix a = matrix::from_host<uint16_t>({8, 24}, halfs(8 * 24, 13, 4.0f), dtype::Float16);
        matrix s = matrix::scalar(1);
        emit(man, "f16_max_i32", MAX, a, s, matrix::max(a, s));
    }
    {   // equal(i16, u16) -> Int32 (1 / 0)
        std::vector<int16_t> x = ints<int16_t>(200, 14, -3, 3);
        std::vector<uint16_t> y = ints<uint16_t>(200, 15, 0, 3);
        matrix a = matrix::from_host<int16_t>({200}, x), b = matrix::from_host<uint16_t>({200}, y);
        emit(man, "i16_eq_u16", EQ, a, b, matrix::equal(a, b));
    }
    {   // bool + bf16 -> BFloat16
        matrix a = matrix::from_host<uint8_t>({64}, ints<uint8_t>(64, 16, 0, 1), dtype::Bool);
        std::vector<uint16_t> h = halfs(64, 17, 3.0f);     // binary16 bits reused as arbitrary bf16 bits
        matrix b = matrix::from_host<uint16_t>({64}, h, dtype::BFloat16);
        emit(man, "bool_add_bf16", ADD, a, b, a + b);
    }
    man.close();
    EXPECT(man.good(), "manifest write failed");
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    if (mode == "cpu") {
        run("promote_types_table", promote_types_table);
        run("scalar_operand_types", scalar_operand_types);
        run("graph_result_dtypes", graph_result_dtypes);
    } else if (mode == "gpu" && argc > 2) {
        g_dir = argv[2];
        run("gpu_mixed_graphs", gpu_mixed_graphs);
    } else {
        std::fprintf(stderr, "usage: dtype_test cpu | gpu <dir>\n");
        return 2;
    }
    return g_fail ? 1 : 0;
}

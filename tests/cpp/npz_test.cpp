// npz_test.cpp -- drives matrix::save_as_npz / matrix::load_npz for tests/test_npz.py.
//
//   npz_test write OUT            every dtype with a numpy descr, as host leaves of fixed shapes
//                                 holding pattern bytes, plus a transposed view of one -> OUT
//   npz_test bf16 OUT             save_as_npz of a BFloat16 leaf must throw (exit 0 if it does)
//   npz_test resave IN OUT        load_npz(IN) then save_as_npz of the loaded leaves -> OUT;
//                                 prints each entry's name and dtype code
//   npz_test load IN              load_npz(IN); prints the error and exits 3 if it throws
//   npz_test gpu IN OUT           a = IN[0], b = IN[1] (float32): saves a + b, a * b, (a + b)^T
//                                 (a view of a device result) and b - a computed on the GPU
//
// Pattern bytes (shared with the Python side): byte k of entry i is (131 k + 17 i + 7) mod 256,
// and for Bool entries that value mod 2.
#include "../../matrix_amd/host/matrix.hpp"

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

static matrix pattern_leaf(const std::vector<size_m>& shape, dtype t, int i) {
    size_t n = 1;
    for (size_m s : shape) n *= s;
    std::vector<uint8_t> b(n * dtype_size(t));
    for (size_t k = 0; k < b.size(); k++) {
        const uint8_t v = (uint8_t)((131 * k + 17 * (size_t)i + 7) & 0xFF);
        b[k] = t == dtype::Bool ? (uint8_t)(v & 1) : v;
    }
    return matrix::from_bytes(shape, t, b.data());
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: npz_test write|bf16|resave|load|gpu ...\n");
        return 2;
    }
    const std::string mode = argv[1];
    try {
        if (mode == "write") {
            const dtype types[] = {dtype::Float, dtype::Float16, dtype::UInt8, dtype::Int32, dtype::Int16,
                                   dtype::UInt32, dtype::UInt16, dtype::Bool, dtype::Int8, dtype::Complex64,
                                   dtype::Int64, dtype::UInt64};
            const std::vector<std::vector<size_m>> shapes = {{3, 4}, {5}, {}, {2, 3, 4}, {2, 0, 3}, {7, 1},
                                                             {1, 2, 1, 3}, {6}, {4, 4}, {3, 2}, {2, 2, 2}, {9}};
            std::vector<matrix> ms;
            for (int i = 0; i < 12; i++) ms.push_back(pattern_leaf(shapes[i], types[i], i));
            ms.push_back(pattern_leaf({3, 5}, dtype::Int32, 12).transpose({1, 0}));     // a view: packed
            matrix::save_as_npz(ms, argv[2]);
        } else if (mode == "bf16") {
            try {
                matrix::save_as_npz({pattern_leaf({2}, dtype::BFloat16, 0)}, argv[2]);
            } catch (const std::runtime_error& e) {
                std::printf("threw: %s\n", e.what());
                return 0;
            }
            return 1;
        } else if (mode == "resave" && argc >= 4) {
            std::vector<std::string> names;
            std::vector<matrix> ms = matrix::load_npz(argv[2], &names);
            for (size_t i = 0; i < ms.size(); i++) std::printf("%s %d\n", names[i].c_str(), (int)ms[i].type);
            matrix::save_as_npz(ms, argv[3]);
        } else if (mode == "load") {
            try {
                matrix::load_npz(argv[2]);
            } catch (const std::runtime_error& e) {
                std::printf("error: %s\n", e.what());
                return 3;
            }
        } else if (mode == "gpu" && argc >= 4) {
            std::vector<matrix> in = matrix::load_npz(argv[2]);
            if (in.size() < 2) throw std::runtime_error("npz_test gpu: need two arrays");
            matrix& a = in[0];
            matrix& b = in[1];
            matrix s = a + b;
            matrix p = a * b;
            matrix d = b - a;
            matrix st = s.transpose({1, 0});
            matrix::save_as_npz({s, p, st, d}, argv[3]);
        } else {
            std::fprintf(stderr, "npz_test: unknown mode %s\n", mode.c_str());
            return 2;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "npz_test: %s\n", e.what());
        return 1;
    }
    return 0;
}

// io.hpp -- tensor file IO on the gfx950 backend (include/SushiBLAS/io.hpp and
// src/io.cpp of the reference): NumPy .npy files (src/io.cpp:136-235) and raw
// binary dumps (src/io.cpp:99-134).
//
// .npy files are format version 1.0 as NumPy writes them: magic "\x93NUMPY",
// version 1.0, a little-endian uint16 header length, then the dict
// "{'descr': '<f4', 'fortran_order': False, 'shape': (2, 3), }" padded with
// spaces and a newline so the data starts on a 64-byte boundary.  Readers
// accept versions 1.0, 2.0 and 3.0.
//
// Deviations from the reference, on purpose:
//  * load_npy parses the header: the dtype must match the tensor's, the shape
//    must match exactly (the reference only searches the header text for each
//    dimension's digits, io.cpp:214-218), and a C-order file read into a
//    column-major tensor (or the reverse) is reordered instead of copied raw;
//  * non-contiguous views are written and read element by element in their
//    logical order (the reference copies num_elements raw bytes from data());
//  * HALF is '<f2' with 2 bytes per element (the reference writes no descr and
//    4 bytes per element for HALF);
//  * DEVICE tensors are staged through pinned buffers, chunk by chunk, with
//    the HIP copies of one chunk overlapping the file access of the next.
#pragma once

#include <SushiBLAS/tensor.hpp>

#include <cstdio>
#include <string>
#include <vector>

namespace SushiBLAS
{
    class Engine;

    /** @brief Parsed .npy header. */
    struct NpyHeader
    {
        std::string descr;           // e.g. "<f4"
        bool fortran_order = false;
        std::vector<int64_t> shape;
        size_t data_offset = 0;      // first data byte in the file
    };

    class IO
    {
        public:
            explicit IO(Engine& e) : engine_(e) {}

            /** @brief Write `t` as a .npy file (runs pending work first, io.cpp:138). */
            void save_npy(const Tensor& t, const std::string& path);

            /** @brief Read a .npy file into `t`, whose dtype and shape must match. */
            void load_npy(Tensor& t, const std::string& path);

            /** @brief Raw element bytes in the tensor's logical order (io.cpp:99-114). */
            void save_bin(const Tensor& t, const std::string& path);

            /** @brief Read raw element bytes written by save_bin (io.cpp:116-134). */
            void load_bin(Tensor& t, const std::string& path);

            /** @brief The complete .npy preamble (magic .. newline) for a tensor. */
            static std::string npy_header(Core::DataType dtype, Core::Layout layout,
                                          const int64_t* shape, int rank);

            /** @brief Parse the preamble at the start of `bytes` (throws if malformed). */
            static NpyHeader parse_npy_header(const std::string& bytes);

            /** @brief The .npy descr of a dtype ("<f2", "<f4", "<f8", "<c8", "<c16"). */
            static const char* npy_descr(Core::DataType dtype);

            /** @brief Bytes per element of a dtype. */
            static size_t element_bytes(Core::DataType dtype);

        private:
            void write_elements(const Tensor& t, std::FILE* f, const std::string& path,
                                bool fortran);
            void read_elements(Tensor& t, std::FILE* f, const std::string& path, bool fortran);

            Engine& engine_;
    };
} // namespace SushiBLAS

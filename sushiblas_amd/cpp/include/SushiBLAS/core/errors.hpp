// errors.hpp -- the reference's error convention: SB_THROW_IF formats a
// message and throws std::runtime_error (include/SushiBLAS/core/logger.hpp:316-323).
// The reference formats with C++20 <format>; this C++17 build substitutes each
// "{}" in the message with the next argument streamed through operator<<.
#pragma once

#include <sstream>
#include <stdexcept>
#include <string>

namespace SushiBLAS
{
    namespace Core
    {
        inline void format_into(std::ostringstream& os, const char* fmt)
        {
            os << fmt;
        }

        template <typename T, typename... Rest>
        void format_into(std::ostringstream& os, const char* fmt, const T& first, const Rest&... rest)
        {
            for (const char* p = fmt; *p; ++p)
            {
                if (p[0] == '{' && p[1] == '}')
                {
                    os << first;
                    format_into(os, p + 2, rest...);
                    return;
                }
                os << *p;
            }
        }

        template <typename... Args>
        std::string format(const char* fmt, const Args&... args)
        {
            std::ostringstream os;
            format_into(os, fmt, args...);
            return os.str();
        }
    } // namespace Core
} // namespace SushiBLAS

#define SB_THROW_IF(condition, ...)                                                     \
    do                                                                                  \
    {                                                                                   \
        if (condition) throw std::runtime_error(::SushiBLAS::Core::format(__VA_ARGS__)); \
    } while (0)

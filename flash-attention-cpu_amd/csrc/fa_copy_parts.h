// fa_copy_parts.h -- how the host-slice copy pool divides one memcpy.
//
// A copy of n bytes is cut into `parts` consecutive pieces whose boundaries
// sit on 64-byte multiples (each thread then starts on its own cache line).
// The piece length is ceil(n / parts) rounded up to 64, so parts * per >= n
// and the pieces cover [0, n) exactly once; trailing parts may be empty.
// Plain C++ with no HIP dependency: the CPU tests compile it on its own.
#ifndef FA_COPY_PARTS_H
#define FA_COPY_PARTS_H

#include <stddef.h>

// Byte range [*begin, *begin + *len) of part `id` (0 <= id < parts) of an
// n-byte copy; *len == 0 when the part is empty.
inline void fa_copy_part_range(size_t n, int parts, int id, size_t* begin, size_t* len) {
    const size_t per = ((n + (size_t)parts - 1) / (size_t)parts + 63) / 64 * 64;
    const size_t b = per * (size_t)id;
    *begin = b < n ? b : n;
    *len = b < n ? (n - b < per ? n - b : per) : 0;
}

#endif

// Memory-overlap test shared by the kernel entry points and the host
// classes: sets of polynomials of u32 words, polynomials a signed number of
// words apart.
#pragma once

#include <cstdint>

namespace chd {

// No polynomial of set a (num_a polynomials of words_a words, pstride_a
// words apart, of either sign) overlaps any polynomial of set b: each pair
// is checked on its own, so a set whose polynomials lie far apart (or in
// descending order) is judged by the memory it covers, not by its hull.
inline bool sets_disjoint_words(const uint32_t *a, long long pstride_a,
                                int num_a, long long words_a,
                                const uint32_t *b, long long pstride_b,
                                int num_b, long long words_b) {
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a);
  const uintptr_t b0 = reinterpret_cast<uintptr_t>(b);
  for (int i = 0; i < num_a; i++) {
    // two's-complement wrap: a negative stride moves the base down
    const uintptr_t alo = a0 + static_cast<uintptr_t>(4LL * i * pstride_a);
    const uintptr_t ahi = alo + 4ull * static_cast<unsigned long long>(words_a);
    for (int j = 0; j < num_b; j++) {
      const uintptr_t blo = b0 + static_cast<uintptr_t>(4LL * j * pstride_b);
      const uintptr_t bhi =
          blo + 4ull * static_cast<unsigned long long>(words_b);
      if (!(ahi <= blo || bhi <= alo)) return false;
    }
  }
  return true;
}

}  // namespace chd

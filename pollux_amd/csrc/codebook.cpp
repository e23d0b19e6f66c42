// Host-side construction of the 196,561-entry Leech codebook.
//
// Follows castor.py:74-190 (_extended_golay24_words, _leech_minimal_vectors,
// _build_codebook_cpu): the extended [24,12] Golay code from the generator
// x^11+x^9+x^7+x^6+x^5+x+1, the three families of raw vectors of squared norm
// 32, an ascending lexicographic sort with coordinate 0 most significant, and
// the origin prepended at index 0.  The table is kept as raw int8 coordinates;
// every numeric form (fp32, bf16, fp16) is derived from it by a per-value map.
//
// Type-3 rows reproduce the reference exactly: -1 where the codeword has a 1,
// +1 elsewhere, then -3 at the chosen position regardless of that position's
// codeword bit (castor.py:134-141).

#include <algorithm>
#include <array>
#include <cstring>
#include <mutex>
#include <vector>

#include "plx_internal.h"

namespace plx {
namespace {

using Row = std::array<int8_t, kDim>;

uint32_t golay_word(uint32_t msg) {
  // systematic cyclic [23,12] encoding: remainder of msg*x^11 mod g(x)
  const uint32_t g = 0xAE3u;
  uint32_t r = msg << 11;
  for (int bit = 22; bit >= 11; --bit)
    if ((r >> bit) & 1u) r ^= g << (bit - 11);
  const uint32_t w23 = (msg << 11) | r;
  const uint32_t parity = static_cast<uint32_t>(__builtin_popcount(w23)) & 1u;
  return w23 | (parity << 23);
}

std::vector<int8_t> build_table() {
  uint32_t words[4096];
  for (uint32_t m = 0; m < 4096; ++m) words[m] = golay_word(m);

  std::vector<Row> rows;
  rows.reserve(kKissing);
  // type 1: two coordinates at +-4
  for (int i = 0; i < kDim; ++i)
    for (int j = i + 1; j < kDim; ++j)
      for (int a = -4; a <= 4; a += 8)
        for (int b = -4; b <= 4; b += 8) {
          Row r{};
          r[i] = static_cast<int8_t>(a);
          r[j] = static_cast<int8_t>(b);
          rows.push_back(r);
        }
  // type 2: +-2 on an octad, even number of minus signs
  for (uint32_t w : words) {
    if (__builtin_popcount(w) != 8) continue;
    int pos[8], n = 0;
    for (int b = 0; b < kDim; ++b)
      if ((w >> b) & 1u) pos[n++] = b;
    for (uint32_t neg = 0; neg < 256; ++neg) {
      if (__builtin_popcount(neg) & 1) continue;
      Row r{};
      for (int k = 0; k < 8; ++k) r[pos[k]] = ((neg >> k) & 1u) ? -2 : 2;
      rows.push_back(r);
    }
  }
  // type 3: -1 on the codeword's support, +1 off it, then -3 at one position
  for (int p = 0; p < kDim; ++p)
    for (uint32_t w : words) {
      Row r{};
      for (int b = 0; b < kDim; ++b) r[b] = ((w >> b) & 1u) ? -1 : 1;
      r[p] = -3;
      rows.push_back(r);
    }

  std::sort(rows.begin(), rows.end(), [](const Row &x, const Row &y) {
    return std::lexicographical_compare(x.begin(), x.end(), y.begin(), y.end());
  });
  std::vector<int8_t> out(static_cast<size_t>(kCodebook) * kDim, 0);
  if (rows.size() == static_cast<size_t>(kKissing))
    std::memcpy(out.data() + kDim, rows.data(), rows.size() * sizeof(Row));
  else
    out.clear();  // signals a generator failure to the caller
  return out;
}

}  // namespace

const int8_t *codebook_raw_host() {
  static std::once_flag once;
  static std::vector<int8_t> table;
  std::call_once(once, [] { table = build_table(); });
  return table.empty() ? nullptr : table.data();
}

const uint32_t *golay_words_host() {
  static std::once_flag once;
  static std::array<uint32_t, 4096> words;
  std::call_once(once, [] {
    for (uint32_t m = 0; m < 4096; ++m) words[m] = golay_word(m);
  });
  return words.data();
}

float raw_to_f32(int k) {
  float s;
  std::memcpy(&s, &kLeechScaleBits, 4);
  return static_cast<float>(k) * s;
}

}  // namespace plx

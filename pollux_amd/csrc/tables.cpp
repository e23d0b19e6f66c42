// Per-device codebook tables, built once per device and kept until exit.
//
// sw_bf16_tiles  the scoring sweep's codes (plx_internal.h: the 98,304 type-3
//                codes, then one representative per antipodal pair of types
//                1-2, zero-padded) rounded to bf16 exactly as the reference's
//                bf16 casts round them (castor.py:437, autocast at
//                castor.py:552), in the MFMA tile layout of quantize.hip;
//                9216 tiles x 768 B = 7,077,888 B.
// sw_raw_tiles   the same codes' raw integers (exact in bf16), same layout,
//                for the fp32-exact NN-P scoring (7,077,888 B).
// sw_dq          the sweep codes' value-id words (kp_dq's format, below) in
//                sweep order, for the quantizer's rescans (1,769,472 B).
// sw_idx         the codebook row of every sweep code (0 for padding) and
// sw_anti        the codebook row of each representative's antipode, indexed
//                from the pair region's start (589,824 + 196,608 B).
// cb_raw         the raw int8 coordinates of all 196,561 rows (4,717,464 B);
//                decoded per value into fp32 / bf16 / fp16 by the kernels.
// kp_gemv        per code 16 B for the fused dequant-linear: the 24 raw
//                coordinates as signed 4-bit fields, then type (0 origin,
//                1 = +-4 pair, 2 = +-2 octad, 3 = one -3) | position of -3 << 8
//                (3,144,976 B).
// kp_dq          per code 3 words for the dequant kernel: the raw alphabet
//                {0,1,2,4,-4,-3,-2,-1} (there is no +3) as value ids 0..7,
//                word p byte i = id(coord 8p+i) | id(coord 8p+4+i) << 4, the
//                order v_perm_b32 lookups want (2,358,732 B).
// gv_halves      the one-token dequant-GEMV's table (bf16 activations): the
//                161 distinct 4-coordinate halves of the codebook rows' planes
//                as two bf16 pairs each (coordinates 0,1 | 2,3; raw integers,
//                exact in bf16), padded to 168 halves, then for each of the
//                4,961 planes (pl_ids' order) its two half symbols, lo | hi << 8
//                (padded to 4,992); 11,328 B, staged in LDS by the kernel.
// kp_half        per code 8 B for the same kernel on the packed stream: the
//                symbols of its 6 halves (coordinates 4h..4h+3), then its type
//                and the position of its -3 (as in kp_gemv) (1,572,488 B).
// pl_ids         the value-id words of the 4,961 distinct 8-coordinate planes
//                of the codebook rows (19,844 B: staged in LDS by the kernels
//                that read the plane layout),
// pl_nib         the same planes as kp_gemv coordinate words (8 signed 4-bit
//                fields, 19,844 B), for the fp32 dequant-linear kernel, and
// code_planes    per code its 3 plane-layout records (plx_internal.h), for
//                plx_h24_plane_layout (1,572,488 B).
// t3_tiles       the structured type-3 scorer's MFMA A operands: the sign
//                patterns +-s (bf16 0x3EB5 / 0xBEB5) of the 2,048
//                representative Golay words (bit 23 clear, ascending), in the
//                sweep tiles' layout (128 tiles, 98,304 B);
// t3_words       the word of each pattern id: representatives, then their
//                complements (16,384 B);
// t3_rows        the codebook row of the type-3 code with pattern id r and its
//                -3 at position p, [4096][24] (393,216 B).
// t2_tiles       the structured pair scorer's MFMA A operands: the 759 octads
//                (ascending masks) with bf16(2s) = 0.70703125 on their 8
//                positions, in the sweep tiles' layout (48 tiles, the last 9
//                slots zero; 36,864 B);
// t2_pos         each octad's 8 positions, ascending, one byte each (6,144 B);
// t2_rows        the codebook row of the type-2 code on octad o whose minus
//                signs on the octad's positions k = 0..6 (ascending) are the
//                bits of p (the eighth sign: even parity), [759][128]
//                (388,608 B);
// t1_rows        the codebook row of the type-1 code with +-4 at positions
//                i < j, [24][24][4] by minus at i | minus at j << 1 (9,216 B);
// t2_steiner     the octad holding each 5-subset of the 24 positions (every
//                5 positions lie in exactly one octad), by the subset's colex
//                rank C(p0,1) + C(p1,2) + ... + C(p4,5), p0 < ... < p4
//                (42,504 entries, 85,008 B).
// t3_dec         a syndrome decoder of the extended Golay code for
//                t12_kernel's type-3 floor: [0, 4096) the coset leader of
//                each syndrome (a least-weight pattern, the first in order of
//                weight, then colex order of its positions), [4096, 4108) the
//                12 basis words whose parities with a pattern are its
//                syndrome bits (the code is self-dual: every codeword has
//                syndrome 0), [4108, 4132) the syndrome of each single
//                position (16,528 B).

#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "plx_internal.h"

namespace plx {
namespace {

uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

std::mutex g_mu;
DeviceTables g_tables[64];

// dequant value ids (raw k -> id): 0->0 1->1 2->2 4->3 -4->4 -3->5 -2->6 -1->7
const uint32_t kId[9] = {4, 5, 6, 7, 0, 1, 2, 0xFF, 3};

// Value-id word of plane p of a raw row: byte i = id(coord 8p+i) | id(coord 8p+4+i) << 4.
uint32_t plane_ids(const int8_t *r, int p) {
  uint32_t d = 0;
  for (int w = 0; w < 8; ++w) d |= kId[r[8 * p + w] + 4] << (8 * (w % 4) + 4 * (w / 4));
  return d;
}

PlaneTables build_planes() {
  PlaneTables pt;
  const int8_t *raw = codebook_raw_host();
  if (!raw) return pt;
  std::vector<uint32_t> all;
  all.reserve(static_cast<size_t>(kCodebook) * 3);
  for (int code = 0; code < kCodebook; ++code)
    for (int p = 0; p < 3; ++p) all.push_back(plane_ids(raw + static_cast<size_t>(code) * kDim, p));
  std::vector<uint32_t> uniq(all);
  std::sort(uniq.begin(), uniq.end());
  uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
  if (uniq.size() > static_cast<size_t>(kMaxPlanes)) return pt;  // signals a failure (13-bit plane indices)
  pt.code_planes.assign(static_cast<size_t>(kCodebook) * 4, 0);
  for (int code = 0; code < kCodebook; ++code) {
    const int8_t *r = raw + static_cast<size_t>(code) * kDim;
    int nz = 0, pos = 0;
    for (int c = 0; c < kDim; ++c) {
      nz += r[c] != 0;
      if (r[c] == -3) pos = c;
    }
    const uint32_t type = nz == 0 ? 0u : nz == 2 ? 1u : nz == 8 ? 2u : 3u;
    const uint32_t extra[3] = {type, static_cast<uint32_t>(pos) & 7u, static_cast<uint32_t>(pos) >> 3};
    for (int p = 0; p < 3; ++p) {
      const uint32_t w = all[static_cast<size_t>(code) * 3 + p];
      const uint32_t k = static_cast<uint32_t>(std::lower_bound(uniq.begin(), uniq.end(), w) - uniq.begin());
      pt.code_planes[static_cast<size_t>(code) * 4 + p] = static_cast<uint16_t>(k | extra[p] << 13);
    }
  }
  pt.ids = std::move(uniq);
  return pt;
}

int build(int dev, DeviceTables *t) {
  const int8_t *raw = codebook_raw_host();
  if (!raw) return fail(PLX_EINVAL, "codebook generator produced a wrong row count");

  uint16_t bf_of[9];
  for (int k = -4; k <= 4; ++k) bf_of[k + 4] = f32_to_bf16_rne(raw_to_f32(k));

  // sweep order: type-3 rows (a -3 coordinate) in index order, then the lower
  // half of the sorted type-1/2 rows (their antipodes are the upper half,
  // reversed); every antipode relation is checked here
  std::vector<int32_t> sym, sweep, anti;
  sym.reserve(2 * kPairCodes);
  sweep.reserve(static_cast<size_t>(kSweepTiles) * kTileCodes);
  for (int code = 1; code < kCodebook; ++code) {
    const int8_t *r = raw + static_cast<size_t>(code) * kDim;
    bool three = false;
    for (int c = 0; c < kDim; ++c) three |= r[c] == -3;
    if (three)
      sweep.push_back(code);
    else
      sym.push_back(code);
  }
  if (static_cast<int>(sweep.size()) != kType3Codes || static_cast<int>(sym.size()) != 2 * kPairCodes)
    return fail(PLX_EINVAL, "codebook has %zu type-3 and %zu type-1/2 rows", sweep.size(), sym.size());
  for (int k = 0; k < kPairCodes; ++k) {
    const int8_t *a = raw + static_cast<size_t>(sym[k]) * kDim;
    const int8_t *b = raw + static_cast<size_t>(sym[2 * kPairCodes - 1 - k]) * kDim;
    for (int c = 0; c < kDim; ++c)
      if (a[c] != -b[c]) return fail(PLX_EINVAL, "codebook row %d has no antipode at the mirrored rank", sym[k]);
    sweep.push_back(sym[k]);
    anti.push_back(sym[2 * kPairCodes - 1 - k]);
  }
  sweep.resize(static_cast<size_t>(kSweepTiles) * kTileCodes, 0);
  anti.resize(static_cast<size_t>(kSweepTiles - kType3Tiles) * kTileCodes, 0);  // every pair-region position

  std::vector<uint16_t> tiles(static_cast<size_t>(kSweepTiles) * (kTileBytes / 2), 0);
  std::vector<uint16_t> raw_tiles(tiles.size(), 0);
  for (int tile = 0; tile < kSweepTiles; ++tile)
    for (int i = 0; i < kTileCodes; ++i) {
      const int code = sweep[static_cast<size_t>(tile) * kTileCodes + i];
      if (code == 0) continue;  // padding stays zero
      for (int p = 0; p < 3; ++p)
        for (int e = 0; e < 8; ++e) {
          const int k = raw[static_cast<size_t>(code) * kDim + 8 * p + e];
          const size_t at = static_cast<size_t>(tile) * 384 + p * 128 + i * 8 + e;
          tiles[at] = bf_of[k + 4];
          raw_tiles[at] = f32_to_bf16_rne(static_cast<float>(k));
        }
    }

  // structured type-3 tables: representative words, their sign-pattern tiles,
  // and the row of every (pattern, -3 position) code, matched against the
  // codebook's type-3 rows (which must be exactly these 98,304 codes)
  std::vector<uint32_t> reps;
  const uint32_t *golay = golay_words_host();
  for (int m = 0; m < 4096; ++m)
    if (((golay[m] >> 23) & 1u) == 0u) reps.push_back(golay[m]);
  std::sort(reps.begin(), reps.end());
  if (static_cast<int>(reps.size()) != kT3Reps) return fail(PLX_EINVAL, "%zu Golay words with bit 23 clear", reps.size());
  std::vector<uint32_t> t3w(kT3Words);
  for (int r = 0; r < kT3Reps; ++r) {
    t3w[r] = reps[r];
    t3w[r + kT3Reps] = reps[r] ^ 0xFFFFFFu;
  }
  std::vector<uint16_t> t3_tiles(static_cast<size_t>(kT3Tiles) * (kTileBytes / 2), 0);
  for (int r = 0; r < kT3Reps; ++r)
    for (int c = 0; c < kDim; ++c)
      t3_tiles[static_cast<size_t>(r / kTileCodes) * 384 + (c / 8) * 128 + (r % kTileCodes) * 8 + c % 8] =
          bf_of[((reps[r] >> c) & 1u) ? 3 : 5];  // -s where the word has a 1, +s elsewhere
  std::vector<std::pair<uint32_t, uint32_t>> t3key;  // (p << 24 | sign bits off p, row)
  t3key.reserve(kType3Codes);
  for (int i = 0; i < kType3Codes; ++i) {
    const int code = sweep[static_cast<size_t>(i)];
    const int8_t *r = raw + static_cast<size_t>(code) * kDim;
    uint32_t bits = 0, pos = kDim;
    for (int c = 0; c < kDim; ++c) {
      if (r[c] == -3) pos = static_cast<uint32_t>(c);
      else if (r[c] == -1) bits |= 1u << c;
    }
    t3key.emplace_back(pos << 24 | bits, static_cast<uint32_t>(code));
  }
  std::sort(t3key.begin(), t3key.end());
  std::vector<uint32_t> t3rows(static_cast<size_t>(kT3Words) * kDim, 0);
  for (int id = 0; id < kT3Words; ++id)
    for (int pp = 0; pp < kDim; ++pp) {
      const uint32_t key = static_cast<uint32_t>(pp) << 24 | (t3w[id] & ~(1u << pp));
      const auto it = std::lower_bound(t3key.begin(), t3key.end(), std::make_pair(key, 0u));
      if (it == t3key.end() || it->first != key)
        return fail(PLX_EINVAL, "no type-3 codebook row for pattern %d with -3 at %d", id, pp);
      t3rows[static_cast<size_t>(id) * kDim + pp] = it->second;
    }

  // structured pair tables: the octads (from the type-2 rows' supports), their
  // tiles and positions, and the row of every type-2 and type-1 code
  std::vector<uint32_t> oct_masks;
  for (int code = 1; code < kCodebook; ++code) {
    const int8_t *r = raw + static_cast<size_t>(code) * kDim;
    uint32_t m = 0;
    int nz = 0;
    for (int c = 0; c < kDim; ++c)
      if (r[c] != 0) {
        m |= 1u << c;
        ++nz;
      }
    if (nz == 8) oct_masks.push_back(m);
  }
  std::sort(oct_masks.begin(), oct_masks.end());
  oct_masks.erase(std::unique(oct_masks.begin(), oct_masks.end()), oct_masks.end());
  if (static_cast<int>(oct_masks.size()) != kT2Octads) return fail(PLX_EINVAL, "%zu octads", oct_masks.size());
  std::vector<uint16_t> t2_tiles(static_cast<size_t>(kT2Tiles) * (kTileBytes / 2), 0);
  std::vector<uint8_t> t2_pos(static_cast<size_t>(kT2Tiles) * kTileCodes * 8, 0);
  std::vector<uint32_t> t2_rows(static_cast<size_t>(kT2Octads) * 128, 0);
  std::vector<uint32_t> t1_rows(static_cast<size_t>(kDim) * kDim * 4, 0);
  for (int o = 0; o < kT2Octads; ++o) {
    int k = 0;
    for (int c = 0; c < kDim; ++c)
      if ((oct_masks[o] >> c) & 1u) {
        t2_tiles[static_cast<size_t>(o / kTileCodes) * 384 + (c / 8) * 128 + (o % kTileCodes) * 8 + c % 8] = bf_of[2 + 4];
        t2_pos[static_cast<size_t>(o) * 8 + k++] = static_cast<uint8_t>(c);
      }
  }
  std::vector<uint16_t> t2_steiner(static_cast<size_t>(kT2Subsets5), 0xFFFFu);
  {
    auto binom = [](int n, int k) {
      long v = 1;
      for (int i = 0; i < k; ++i) v = v * (n - i) / (i + 1);
      return n < k ? 0L : v;
    };
    for (int o = 0; o < kT2Octads; ++o) {
      const uint8_t *pp = t2_pos.data() + static_cast<size_t>(o) * 8;
      for (int m = 0; m < 256; ++m) {
        if (__builtin_popcount(m) != 5) continue;
        long rank = 0;
        int k = 0;
        for (int b = 0; b < 8; ++b)
          if ((m >> b) & 1) rank += binom(pp[b], ++k);
        if (t2_steiner[static_cast<size_t>(rank)] != 0xFFFFu) return fail(PLX_EINVAL, "5 positions in two octads");
        t2_steiner[static_cast<size_t>(rank)] = static_cast<uint16_t>(o);
      }
    }
    for (uint16_t v : t2_steiner)
      if (v == 0xFFFFu) return fail(PLX_EINVAL, "5 positions in no octad");
  }
  std::vector<uint32_t> t3_dec(static_cast<size_t>(kT3DecWords), 0xFFFFFFFFu);
  {
    // basis: the first 12 words, in table order, independent of those before them (GF(2) elimination:
    // piv[b] holds a reduced word whose leading bit is b)
    const uint32_t *golay = golay_words_host();
    uint32_t basis[12], piv[kDim] = {};
    int nb = 0;
    for (int m = 0; m < 4096 && nb < 12; ++m) {
      uint32_t r = golay[m];
      for (int b = kDim - 1; b >= 0 && r != 0u; --b)
        if (((r >> b) & 1u) != 0u) {
          if (piv[b] == 0u) {
            piv[b] = r;
            basis[nb++] = golay[m];
            break;
          }
          r ^= piv[b];
        }
    }
    if (nb != 12) return fail(PLX_EINVAL, "Golay basis of %d words", nb);
    auto syndrome = [&](uint32_t e) {
      uint32_t sy = 0u;
      for (int j = 0; j < 12; ++j) sy |= static_cast<uint32_t>(__builtin_popcount(e & basis[j]) & 1) << j;
      return sy;
    };
    for (int m = 0; m < 4096; ++m)
      if (syndrome(golay[m]) != 0u) return fail(PLX_EINVAL, "Golay word with a nonzero syndrome");
    // leaders by weight 0..4, positions in colex order within a weight (the covering radius is 4)
    int found = 0;
    for (int wt = 0; wt <= 4 && found < 4096; ++wt) {
      int pos[4] = {0, 1, 2, 3};
      while (true) {
        uint32_t e = 0u;
        for (int k = 0; k < wt; ++k) e |= 1u << pos[k];
        const uint32_t sy = syndrome(e);
        if (t3_dec[sy] == 0xFFFFFFFFu) {
          t3_dec[sy] = e;
          ++found;
        }
        // next combination of wt positions in colex order
        int k = 0;
        while (k < wt && pos[k] + 1 == (k + 1 < wt ? pos[k + 1] : kDim)) ++k;
        if (k == wt) break;
        ++pos[k];
        for (int i = 0; i < k; ++i) pos[i] = i;
      }
    }
    if (found != 4096) return fail(PLX_EINVAL, "Golay syndromes without a leader of weight <= 4: %d", 4096 - found);
    for (int j = 0; j < 12; ++j) t3_dec[4096 + j] = basis[j];
    for (int c = 0; c < kDim; ++c) t3_dec[4108 + c] = syndrome(1u << c);
  }
  int n_t2 = 0, n_t1 = 0;
  for (int code = 1; code < kCodebook; ++code) {
    const int8_t *r = raw + static_cast<size_t>(code) * kDim;
    uint32_t m = 0, minus = 0;
    int nz = 0, lo = -1, hi = -1;
    for (int c = 0; c < kDim; ++c)
      if (r[c] != 0) {
        if (r[c] < 0) minus |= 1u << nz;
        m |= 1u << c;
        lo = lo < 0 ? c : lo;
        hi = c;
        ++nz;
      }
    if (nz == 8) {
      const int o = static_cast<int>(std::lower_bound(oct_masks.begin(), oct_masks.end(), m) - oct_masks.begin());
      if (o >= kT2Octads || oct_masks[o] != m || (__builtin_popcount(minus) & 1) != 0)
        return fail(PLX_EINVAL, "codebook row %d is no even-sign octad code", code);
      uint32_t &slot = t2_rows[static_cast<size_t>(o) * 128 + (minus & 0x7Fu)];
      if (slot != 0) return fail(PLX_EINVAL, "two octad codes share a sign pattern (row %d)", code);
      slot = static_cast<uint32_t>(code);
      ++n_t2;
    } else if (nz == 2) {
      uint32_t &slot = t1_rows[(static_cast<size_t>(lo) * kDim + hi) * 4 + minus];
      if (slot != 0) return fail(PLX_EINVAL, "two type-1 codes share positions and signs (row %d)", code);
      slot = static_cast<uint32_t>(code);
      ++n_t1;
    }
  }
  if (n_t2 != kT2Octads * 128 || n_t1 != 276 * 4) return fail(PLX_EINVAL, "%d type-2 and %d type-1 rows", n_t2, n_t1);

  // dequant-linear entries: 24 signed 4-bit coordinates, then type | pos << 8
  std::vector<uint32_t> gemv(static_cast<size_t>(kCodebook) * 4, 0);
  std::vector<uint32_t> dq(static_cast<size_t>(kCodebook) * 3, 0);
  // the distinct 4-coordinate halves (key: the 4 raw values as bytes), ascending
  auto half_key = [](const int8_t *c) {
    uint32_t k = 0;
    for (int i = 0; i < 4; ++i) k |= static_cast<uint32_t>(static_cast<uint8_t>(c[i] + 4)) << (8 * (3 - i));
    return k;
  };
  std::vector<uint32_t> halves;
  for (int code = 0; code < kCodebook; ++code)
    for (int h = 0; h < 6; ++h) halves.push_back(half_key(raw + static_cast<size_t>(code) * kDim + 4 * h));
  std::sort(halves.begin(), halves.end());
  halves.erase(std::unique(halves.begin(), halves.end()), halves.end());
  if (static_cast<int>(halves.size()) > kGvHalves) return fail(PLX_EINVAL, "%zu distinct codebook halves", halves.size());
  auto half_sym = [&](const int8_t *c) {
    return static_cast<uint32_t>(std::lower_bound(halves.begin(), halves.end(), half_key(c)) - halves.begin());
  };
  std::vector<uint32_t> gv(static_cast<size_t>(kGvVecs) * 4, 0);
  for (size_t k = 0; k < halves.size(); ++k) {
    uint16_t b[4];
    for (int i = 0; i < 4; ++i) b[i] = f32_to_bf16_rne(static_cast<float>(static_cast<int>((halves[k] >> (8 * (3 - i))) & 0xFFu) - 4));
    gv[2 * k] = b[0] | static_cast<uint32_t>(b[1]) << 16;
    gv[2 * k + 1] = b[2] | static_cast<uint32_t>(b[3]) << 16;
  }
  std::vector<uint32_t> kp_half(static_cast<size_t>(kCodebook) * 2, 0);
  for (int code = 0; code < kCodebook; ++code) {
    const int8_t *r = raw + static_cast<size_t>(code) * kDim;
    uint32_t *e = gemv.data() + static_cast<size_t>(code) * 4;
    uint32_t *d = dq.data() + static_cast<size_t>(code) * 3;
    int nz = 0, pos = 0;
    for (int c = 0; c < kDim; ++c) {
      e[c / 8] |= (static_cast<uint32_t>(r[c]) & 0xFu) << (4 * (c % 8));
      nz += r[c] != 0;
      if (r[c] == -3) pos = c;
      const uint32_t id = kId[r[c] + 4];
      if (id > 7) return fail(PLX_EINVAL, "codebook coordinate %d outside the dequant alphabet", r[c]);
      const int p = c / 8, w = c % 8;
      d[p] |= id << (8 * (w % 4) + 4 * (w / 4));
    }
    const uint32_t type = nz == 0 ? 0u : nz == 2 ? 1u : nz == 8 ? 2u : 3u;
    e[3] = type | (static_cast<uint32_t>(pos) << 8);
    uint32_t *o = kp_half.data() + static_cast<size_t>(code) * 2;
    for (int h = 0; h < 6; ++h) o[h / 4] |= half_sym(r + 4 * h) << (8 * (h % 4));
    o[1] |= type << 16 | static_cast<uint32_t>(pos) << 24;
  }

  struct Upload {
    const void *host;
    size_t bytes;
    void **dev;
  };
  std::vector<uint32_t> sw_dq(sweep.size() * 3, 0);
  for (size_t i = 0; i < sweep.size(); ++i)
    for (int p = 0; p < 3; ++p) sw_dq[i * 3 + p] = dq[static_cast<size_t>(sweep[i]) * 3 + p];

  void *dt = nullptr, *drt = nullptr, *dsq = nullptr, *dsi = nullptr, *dsa = nullptr, *dr = nullptr, *dg = nullptr,
       *dd = nullptr, *dk = nullptr, *dpi = nullptr, *dcp = nullptr, *dpn = nullptr, *d3t = nullptr, *d3w = nullptr,
       *d3r = nullptr, *dgv = nullptr, *d2t = nullptr, *d2p = nullptr, *d2r = nullptr, *d1r = nullptr,
       *d2s = nullptr, *d3d = nullptr;
  const PlaneTables *pt = plane_tables_host();
  if (!pt) return fail(PLX_EINVAL, "the codebook rows take more than %d distinct planes", kMaxPlanes);
  std::vector<uint32_t> pl_pad(pt->ids);  // whole 16-byte vectors (the kernels stage it by uint4)
  pl_pad.resize((pl_pad.size() + 3) & ~static_cast<size_t>(3), 0u);
  // value id -> raw value (kId's inverse), then the plane's coordinates as signed nibbles
  static const int kIdValue[8] = {0, 1, 2, 4, -4, -3, -2, -1};
  std::vector<uint32_t> pl_nib(pl_pad.size(), 0u);
  for (size_t k = 0; k < pt->ids.size(); ++k)
    for (int w = 0; w < 8; ++w) {
      const uint32_t id = (pt->ids[k] >> (8 * (w % 4) + 4 * (w / 4))) & 0xFu;
      pl_nib[k] |= (static_cast<uint32_t>(kIdValue[id & 7u]) & 0xFu) << (4 * w);
    }
  // each plane's two half symbols (the plane's value ids decoded to raw values)
  {
    if (pt->ids.size() > static_cast<size_t>(kGvPlanes)) return fail(PLX_EINVAL, "%zu planes", pt->ids.size());
    uint16_t *ph = reinterpret_cast<uint16_t *>(gv.data() + 2 * kGvHalves);
    for (size_t k = 0; k < pt->ids.size(); ++k) {
      int8_t c[8];
      for (int w = 0; w < 8; ++w) c[w] = static_cast<int8_t>(kIdValue[(pt->ids[k] >> (8 * (w % 4) + 4 * (w / 4))) & 7u]);
      ph[k] = static_cast<uint16_t>(half_sym(c) | half_sym(c + 4) << 8);
    }
  }
  const Upload ups[] = {
      {tiles.data(), tiles.size() * 2, &dt},
      {raw_tiles.data(), raw_tiles.size() * 2, &drt},
      {sw_dq.data(), sw_dq.size() * 4, &dsq},
      {sweep.data(), sweep.size() * 4, &dsi},
      {anti.data(), anti.size() * 4, &dsa},
      {raw, static_cast<size_t>(kCodebook) * kDim, &dr},
      {gemv.data(), gemv.size() * 4, &dg},
      {dq.data(), dq.size() * 4, &dd},
      {kp_half.data(), kp_half.size() * 4, &dk},
      {gv.data(), gv.size() * 4, &dgv},
      {pl_pad.data(), pl_pad.size() * 4, &dpi},
      {pt->code_planes.data(), pt->code_planes.size() * 2, &dcp},
      {pl_nib.data(), pl_nib.size() * 4, &dpn},
      {t3_tiles.data(), t3_tiles.size() * 2, &d3t},
      {t3w.data(), t3w.size() * 4, &d3w},
      {t3rows.data(), t3rows.size() * 4, &d3r},
      {t2_tiles.data(), t2_tiles.size() * 2, &d2t},
      {t2_pos.data(), t2_pos.size(), &d2p},
      {t2_rows.data(), t2_rows.size() * 4, &d2r},
      {t1_rows.data(), t1_rows.size() * 4, &d1r},
      {t2_steiner.data(), t2_steiner.size() * 2, &d2s},
      {t3_dec.data(), t3_dec.size() * 4, &d3d},
  };
  int st = PLX_OK;
  for (const Upload &u : ups) {
    if (hipMalloc(u.dev, u.bytes) != hipSuccess) {
      *u.dev = nullptr;
      st = fail(PLX_ENOMEM, "device table allocation (%zu B) failed on device %d", u.bytes, dev);
      break;
    }
    st = check_hip(hipMemcpy(*u.dev, u.host, u.bytes, hipMemcpyHostToDevice), "upload codebook table");
    if (st != PLX_OK) break;
  }
  if (st != PLX_OK) {
    for (const Upload &u : ups)
      if (*u.dev) (void)hipFree(*u.dev);
    return st;
  }
  t->sw_bf16_tiles = static_cast<uint8_t *>(dt);
  t->sw_raw_tiles = static_cast<uint8_t *>(drt);
  t->sw_dq = static_cast<uint32_t *>(dsq);
  t->sw_idx = static_cast<uint32_t *>(dsi);
  t->sw_anti = static_cast<uint32_t *>(dsa);
  t->cb_raw = static_cast<int8_t *>(dr);
  t->kp_gemv = static_cast<uint8_t *>(dg);
  t->kp_dq = static_cast<uint32_t *>(dd);
  t->kp_half = static_cast<uint2 *>(dk);
  t->gv_tab = static_cast<uint4 *>(dgv);
  t->pl_ids = static_cast<uint32_t *>(dpi);
  t->code_planes = static_cast<uint16_t *>(dcp);
  t->pl_nib = static_cast<uint32_t *>(dpn);
  t->t3_tiles = static_cast<uint8_t *>(d3t);
  t->t3_words = static_cast<uint32_t *>(d3w);
  t->t3_rows = static_cast<uint32_t *>(d3r);
  t->t2_tiles = static_cast<uint8_t *>(d2t);
  t->t2_pos = static_cast<uint2 *>(d2p);
  t->t2_rows = static_cast<uint32_t *>(d2r);
  t->t1_rows = static_cast<uint32_t *>(d1r);
  t->t2_steiner = static_cast<uint16_t *>(d2s);
  t->t3_dec = static_cast<uint32_t *>(d3d);
  t->device = dev;
  return PLX_OK;
}

}  // namespace

const PlaneTables *plane_tables_host() {
  static std::once_flag once;
  static PlaneTables pt;
  std::call_once(once, [] { pt = build_planes(); });
  return pt.ids.empty() ? nullptr : &pt;
}

int get_tables(const DeviceTables **out) {
  int dev = 0;
  int st = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (st != PLX_OK) return st;
  if (dev < 0 || dev >= 64) return fail(PLX_EINVAL, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceTables *t = &g_tables[dev];
  if (t->device != dev) {
    st = build(dev, t);
    if (st != PLX_OK) return st;
  }
  *out = t;
  return PLX_OK;
}

int get_tables_built(const DeviceTables **out) {
  int dev = 0;
  int st = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (st != PLX_OK) return st;
  if (dev < 0 || dev >= 64) return fail(PLX_EINVAL, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_mu);
  const DeviceTables *t = &g_tables[dev];
  if (t->device != dev)
    return fail(PLX_EINVAL, "the codebook tables of device %d are not built: call plx_device_init() on it first", dev);
  *out = t;
  return PLX_OK;
}

}  // namespace plx

// Order of the row reads of the wide-bundle kernel's literal stream, shared
// by the host binding (search_plan.cpp) and the device binding kernel
// (bloom_search.hip), which must agree word for word.
//
// The wide-bundle kernel stages 64 bytes of every bundle row in LDS (a
// slice tile), and the four lanes of a quad read one 64-byte row per
// ds_read_b128.  The LDS serves 16 lanes (four quads) of such a read per
// pass, 256 bytes across its banks, so a row's bank group is its index
// mod 4: four rows with distinct residues take one pass, and rows sharing a
// residue take one pass each.  The four quads of a 16-lane group evaluate
// four records of one round step (one record each), reading position k of
// their records in read k.  A record's positions are ANDed, so their order
// is free: balance_wide_choice and balance_source permute each record's
// positions so that the residues of each read are spread over the bank
// groups.  With random rows the expected passes per read drop from 2.13 to
// about 1.66 (K = 4).
#pragma once

#include <cstdint>

#include "search_plan.hpp"
#include "st_common.hpp"

namespace st {

constexpr int kBalanceMaxK = 7;    // positions of a wide-kernel record (k <= 7)
constexpr int kBalanceRecords = 4; // records read together by 16 lanes

// LDS bank group of a slice-tile position (a byte offset row * 64).
ST_HD uint32_t wide_bank_group(uint32_t pos) { return (pos / kWideSliceBytes) & 3u; }

// Greedy per read k: the records pick in increasing order of the number of
// distinct residues they have left (ties: record order); each takes the
// residue used least in this read so far, then the one with the most rows
// left over the four records, then the smallest.  res[i] holds the residue
// of record i's position j in bits 2j, 2j + 1 (j < ks); choice[i] receives
// the residue record i reads in read k in bits 2k, 2k + 1.
ST_HD void balance_wide_choice(const uint32_t (&res)[kBalanceRecords], int ks,
                               uint32_t (&choice)[kBalanceRecords]) {
  uint32_t cnt[kBalanceRecords];  // rows left per residue, 8 bits each
#pragma unroll
  for (int i = 0; i < kBalanceRecords; ++i) {
    cnt[i] = 0;
    for (int j = 0; j < ks; ++j) cnt[i] += 1u << (8 * ((res[i] >> (2 * j)) & 3u));
    choice[i] = 0;
  }
  for (int k = 0; k < ks; ++k) {
    const uint32_t deg = cnt[0] + cnt[1] + cnt[2] + cnt[3];
    int distinct[kBalanceRecords];
#pragma unroll
    for (int i = 0; i < kBalanceRecords; ++i) {
      int d = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) d += ((cnt[i] >> (8 * c)) & 0xFFu) != 0u;
      distinct[i] = d;
    }
    uint32_t used = 0;
#pragma unroll
    for (int step = 0; step < kBalanceRecords; ++step) {
#pragma unroll
      for (int i = 0; i < kBalanceRecords; ++i) {
        int rank = 0;
#pragma unroll
        for (int o = 0; o < kBalanceRecords; ++o)
          rank += distinct[o] < distinct[i] || (distinct[o] == distinct[i] && o < i);
        if (rank != step) continue;
        int best = -1;
        uint32_t bu = 0, bd = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (((cnt[i] >> (8 * c)) & 0xFFu) == 0u) continue;
          const uint32_t u = (used >> (8 * c)) & 0xFFu, d = (deg >> (8 * c)) & 0xFFu;
          if (best < 0 || u < bu || (u == bu && d > bd)) {
            best = c;
            bu = u;
            bd = d;
          }
        }
        choice[i] |= static_cast<uint32_t>(best) << (2 * k);
        cnt[i] -= 1u << (8 * best);
        used += 1u << (8 * best);
      }
    }
  }
}

// Source of read k of a record: its n-th position (in order) with the
// residue read k takes, n the earlier reads that take that residue.
ST_HD int balance_source(uint32_t res, uint32_t choice, int k, int ks) {
  const uint32_t c = (choice >> (2 * k)) & 3u;
  int n = 0;
  for (int e = 0; e < k; ++e) n += ((choice >> (2 * e)) & 3u) == c;
  for (int j = 0; j < ks; ++j) {
    if (((res >> (2 * j)) & 3u) != c) continue;
    if (n == 0) return j;
    --n;
  }
  return k;  // not reached: read k's residue has a row left
}

// Whether the stream of a plan with ks positions per record gets balanced
// units (a record of the wide-bundle kernel holds 2 .. 7 positions).
ST_HD bool balance_applies(int ks) { return ks >= 2 && ks <= kBalanceMaxK; }

}  // namespace st

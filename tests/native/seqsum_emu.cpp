// seqsum_emu.cpp -- host emulation of the work-group algorithm in
// cudaforge_amd/csrc/seqsum.hpp (same helpers, lanes replaced by loops).
// TEST INFRASTRUCTURE: fuzzed against a plain sequential fp32 loop.
#include <cstdint>
#include <vector>

#include "../../cudaforge_amd/csrc/seqsum.hpp"

using namespace cfa::seq;

namespace {

struct Emu {
  int nt, tile, nw;
  float delta;
  std::vector<float> x;      // staged block
  std::vector<uint32_t> tI;  // per tile
  std::vector<int> treg;
  std::vector<uint32_t> wI;
  std::vector<int> wreg;
  long long serial_tiles = 0;

  long long serial_tile(int t, float &s, bool cdf, float r, long long blk0) {
    ++serial_tiles;
    for (int k = 0; k < tile; ++k) {
      s = s + x[(size_t)t * tile + k];
      if (cdf && r <= s) return blk0 + (long long)t * tile + k;
    }
    return -1;
  }

  // generic run walker over items [first, first+count) with per-item (I, reg)
  template <class GetI, class GetReg, class OnHit, class OnBad>
  long long walk(int count, float &s, bool cdf, float r, GetI getI, GetReg getReg, OnHit onhit,
                 OnBad onbad) {
    int t = 0;
    while (t < count) {
      int rs = region_of(s);
      uint32_t a = units_of(s, rs);
      // longest valid prefix from t
      uint32_t inc = 0;
      int nvalid = 0;
      for (int L = t; L < count && L - t < 64; ++L) {
        uint32_t v = getI(L);
        bool vin = v != kBad && getReg(L) == rs;
        if (!vin) break;
        if (a + inc + v > kUnitsTop) break;
        if (cdf && r <= value_of(a + inc + v, rs)) {
          s = value_of(a + inc, rs);
          return onhit(L, s);
        }
        inc += v;
        ++nvalid;
      }
      if (nvalid > 0) {
        s = value_of(a + inc, rs);
        t += nvalid;
        continue;
      }
      long long f = onbad(t, s);
      if (f >= 0) return f;
      ++t;
    }
    return -1;
  }

  long long tile_sweep(int w, float &s, bool cdf, float r, long long blk0) {
    return walk(
        64, s, cdf, r, [&](int L) { return tI[w * 64 + L]; }, [&](int L) { return treg[w * 64 + L]; },
        [&](int L, float &ss) { return serial_tile(w * 64 + L, ss, cdf, r, blk0); },
        [&](int L, float &ss) { return serial_tile(w * 64 + L, ss, cdf, r, blk0); });
  }

  long long sweep_block(float &s, bool cdf, float r, long long blk0) {
    return walk(
        nw, s, cdf, r, [&](int L) { return wI[L]; }, [&](int L) { return wreg[L]; },
        [&](int L, float &ss) { return tile_sweep(L, ss, cdf, r, blk0); },
        [&](int L, float &ss) { return tile_sweep(L, ss, cdf, r, blk0); });
  }
};

}  // namespace

extern "C" int emu_seq(const float *xin, long long n, int cdf, float r, int nt, float delta,
                       float *out_sum, long long *out_idx, long long *out_serial) {
  Emu e;
  e.nt = nt;
  e.tile = 16;
  e.nw = nt / 64;
  e.delta = delta;
  const int blk = nt * 16;
  e.x.resize(blk);
  e.tI.resize(nt);
  e.treg.resize(nt);
  e.wI.resize(e.nw);
  e.wreg.resize(e.nw);
  float s = 0.0f;
  long long found = -1;
  for (long long blk0 = 0; blk0 < n && found < 0; blk0 += blk) {
    for (int m = 0; m < blk; ++m) e.x[m] = (blk0 + m < n) ? xin[blk0 + m] : 0.0f;
    // approximate prefix: fp32 tile sums, wave inclusive scans, wave prefixes
    std::vector<float> A(nt);
    for (int t = 0; t < nt; ++t) {
      float a = 0.0f;
      for (int k = 0; k < 16; ++k) a += e.x[(size_t)t * 16 + k];
      A[t] = a;
    }
    std::vector<float> wtot(e.nw);
    std::vector<float> incl(nt);
    for (int w = 0; w < e.nw; ++w) {
      float c = 0.0f;
      for (int l = 0; l < 64; ++l) {
        c += A[w * 64 + l];
        incl[w * 64 + l] = c;
      }
      wtot[w] = c;
    }
    for (int t = 0; t < nt; ++t) {
      int w = t / 64;
      float wpre = 0.0f;
      for (int q = 0; q < w; ++q) wpre += wtot[q];
      float E = s + (wpre + (incl[t] - A[t]));
      int rlo = region_of(E * (1.0f - delta));
      int rhi = region_of((E + A[t]) * (1.0f + delta));
      bool ok = rlo == rhi;
      uint32_t I0 = kBad, I1 = kBad;
      if (ok) {
        quantize_tile(&e.x[(size_t)t * 16], 16, rlo, I0, I1);
        ok = (I0 == I1) && I0 <= kUnitsTop;
      }
      e.tI[t] = ok ? I0 : kBad;
      e.treg[t] = rlo;
    }
    for (int w = 0; w < e.nw; ++w) {
      bool uni = true;
      uint32_t tot = 0;
      for (int l = 0; l < 64; ++l) {
        uint32_t v = e.tI[w * 64 + l];
        if (v == kBad || e.treg[w * 64 + l] != e.treg[w * 64]) uni = false;
        else tot += v;
      }
      e.wI[w] = uni ? (tot < kSat ? tot : kSat) : kBad;
      e.wreg[w] = e.treg[w * 64];
    }
    found = e.sweep_block(s, cdf != 0, r, blk0);
  }
  *out_sum = s;
  *out_idx = found;
  *out_serial = e.serial_tiles;
  return 0;
}

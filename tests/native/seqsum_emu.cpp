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
  std::vector<Inc> tI;  // per tile
  std::vector<int> treg;
  std::vector<Inc> wI;
  std::vector<int> wreg;
  std::vector<int> wserial;
  long long serial_tiles = 0;

  long long serial_tile(int t, float &s, bool cdf, float r, long long blk0) {
    ++serial_tiles;
    for (int k = 0; k < tile; ++k) {
      s = s + x[(size_t)t * tile + k];
      if (cdf && r <= s) return blk0 + (long long)t * tile + k;
    }
    return -1;
  }

  // the device walk: up to 64 items per step, composed in lane order, the
  // valid prefix applied at once; an invalid first item is descended into
  template <class GetI, class GetReg, class Descend>
  long long walk(int count, float &s, bool cdf, float r, GetI getI, GetReg getReg,
                 Descend descend) {
    int t = 0;
    while (t < count) {
      int rs = region_of(s);
      uint32_t a = units_of(s, rs);
      Inc acc = inc_identity();
      int nvalid = 0;
      for (int L = t; L < count && L - t < 64; ++L) {
        Inc v = getI(L);
        bool vin = v.e != kBad && (getReg(L) == rs || getReg(L) == kAnyRegion);
        if (!vin) break;
        Inc nxt = compose(acc, v);
        uint32_t inc = inc_at(nxt, a);
        if (a + inc > kUnitsTop) break;
        if (cdf && r <= value_of(a + inc, rs)) {
          s = value_of(a + inc_at(acc, a), rs);
          return descend(L, s);
        }
        acc = nxt;
        ++nvalid;
      }
      if (nvalid > 0) {
        s = value_of(a + inc_at(acc, a), rs);
        t += nvalid;
        continue;
      }
      long long f = descend(t, s);
      if (f >= 0) return f;
      ++t;
    }
    return -1;
  }

  long long tile_sweep(int w, float &s, bool cdf, float r, long long blk0) {
    return walk(
        64, s, cdf, r, [&](int L) { return tI[w * 64 + L]; }, [&](int L) { return treg[w * 64 + L]; },
        [&](int L, float &ss) { return serial_tile(w * 64 + L, ss, cdf, r, blk0); });
  }

  // a wave with several straddling tiles is replayed element by element
  long long serial_wave(int w, float &s, bool cdf, float r, long long blk0) {
    for (int k = 0; k < 64 * tile; ++k) {
      s = s + x[(size_t)w * 64 * tile + k];
      if (cdf && r <= s) return blk0 + (long long)w * 64 * tile + k;
    }
    return -1;
  }

  long long sweep_block(float &s, bool cdf, float r, long long blk0) {
    return walk(
        nw, s, cdf, r, [&](int L) { return wI[L]; }, [&](int L) { return wreg[L]; },
        [&](int L, float &ss) {
          return wserial[L] ? serial_wave(L, ss, cdf, r, blk0) : tile_sweep(L, ss, cdf, r, blk0);
        });
  }
};

}  // namespace

extern "C" int emu_seq(const float *xin, long long n, int cdf, float r, int nt, float delta,
                       float *out_sum, long long *out_idx, long long *out_serial) {
  Emu e;
  e.nt = nt;
  e.tile = 16;
  e.nw = nt / 64;
  e.delta = delta > 0.0f ? delta : kDelta;
  const int blk = nt * 16;
  e.x.resize(blk);
  e.tI.resize(nt);
  e.treg.resize(nt);
  e.wI.resize(e.nw);
  e.wreg.resize(e.nw);
  e.wserial.resize(e.nw);
  std::vector<int> straddle(nt);
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
      Inc f{kBad, kBad};
      if (A[t] == 0.0f) {
        ok = true;
        rlo = kAnyRegion;
        f = inc_identity();
      } else if (ok) {
        quantize_tile(&e.x[(size_t)t * 16], 16, rlo, f.e, f.o);
        ok = f.e <= kUnitsTop && f.o <= kUnitsTop;
        if (!ok) f = Inc{kBad, kBad};
      }
      e.tI[t] = f;
      e.treg[t] = rlo;
      straddle[t] = (!ok && A[t] != 0.0f) ? 1 : 0;
    }
    for (int w = 0; w < e.nw; ++w) {
      bool uni = true;
      Inc tot = inc_identity();
      int r0 = kAnyRegion;
      for (int l = 0; l < 64; ++l)
        if (e.treg[w * 64 + l] != kAnyRegion) { r0 = e.treg[w * 64 + l]; break; }
      for (int l = 0; l < 64; ++l) {
        Inc v = e.tI[w * 64 + l];
        int rg = e.treg[w * 64 + l];
        if (v.e == kBad || (rg != r0 && rg != kAnyRegion)) uni = false;
        else tot = compose(tot, v);
      }
      e.wI[w] = uni ? tot : Inc{kBad, kBad};
      e.wreg[w] = r0;
      int crossings = 0;
      for (int l = 0; l < 64; ++l) crossings += straddle[w * 64 + l];
      e.wserial[w] = crossings >= kSerialCrossings ? 1 : 0;
    }
    found = e.sweep_block(s, cdf != 0, r, blk0);
  }
  *out_sum = s;
  *out_idx = found;
  *out_serial = e.serial_tiles;
  return 0;
}

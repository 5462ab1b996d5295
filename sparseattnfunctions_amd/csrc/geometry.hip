// Host-side, data-independent layout tables of the CogVideoX token grid: the static local
// 3-D window of the combined mask. Computed once per geometry on the CPU and uploaded by
// the caller; no GPU state is touched here.
#include <algorithm>
#include <cstring>

#include "sa_common.h"

namespace {

struct VideoPos {
  bool video;
  int t, h, w;
};

// Token index -> (t, h, w) of the video grid (text first, then row-major t, h, w).
VideoPos token_pos(int token, int text_len, int Hp, int Wp) {
  VideoPos p{false, 0, 0, 0};
  if (token < text_len) return p;
  const int v = token - text_len;
  p.video = true;
  p.t = v / (Hp * Wp);
  p.h = (v / Wp) % Hp;
  p.w = v % Wp;
  return p;
}

inline int iabs(int x) { return x < 0 ? -x : x; }

}  // namespace

extern "C" int sa_local_window_bitmap(int L, int block, int text_len, int T, int Hp, int Wp, int dt, int dh,
                                      int dw, uint8_t* bitmap) {
  SA_REQUIRE(bitmap, "sa_local_window_bitmap: null bitmap");
  SA_REQUIRE(block > 0 && text_len >= 0 && T > 0 && Hp > 0 && Wp > 0 && dt >= 0 && dh >= 0 && dw >= 0,
             "sa_local_window_bitmap: bad geometry");
  SA_REQUIRE(L == text_len + T * Hp * Wp, "sa_local_window_bitmap: L=%d != text_len + T*Hp*Wp", L);
  const int nb = sa::cdiv(L, block);
  // Each block is represented by its centre token (clamped to the last token).
  for (int qb = 0; qb < nb; ++qb) {
    const VideoPos pq = token_pos(std::min(qb * block + block / 2, L - 1), text_len, Hp, Wp);
    for (int kb = 0; kb < nb; ++kb) {
      const VideoPos pk = token_pos(std::min(kb * block + block / 2, L - 1), text_len, Hp, Wp);
      const bool on = pq.video && pk.video && iabs(pq.t - pk.t) <= dt && iabs(pq.h - pk.h) <= dh &&
                      iabs(pq.w - pk.w) <= dw;
      bitmap[(int64_t)qb * nb + kb] = on ? 1 : 0;
    }
  }
  return sa::ok();
}

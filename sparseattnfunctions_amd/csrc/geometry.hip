// Host-side, data-independent layout tables of the CogVideoX token grid: the static local
// 3-D window of the combined mask. Computed once per geometry on the CPU and uploaded by
// the caller; no GPU state is touched here.
#include <algorithm>
#include <cstring>
#include <vector>

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

extern "C" int sa_local_window_bitmap_perm(int L, int block, int text_len, int T, int Hp, int Wp, int dt, int dh,
                                           int dw, const int32_t* perm, uint8_t* bitmap) {
  SA_REQUIRE(bitmap && perm, "sa_local_window_bitmap_perm: null pointer");
  SA_REQUIRE(block > 0 && text_len >= 0 && T > 0 && Hp > 0 && Wp > 0 && dt >= 0 && dh >= 0 && dw >= 0,
             "sa_local_window_bitmap_perm: bad geometry");
  SA_REQUIRE(L == text_len + T * Hp * Wp, "sa_local_window_bitmap_perm: L=%d != text_len + T*Hp*Wp", L);
  const int nb = sa::cdiv(L, block);
  std::vector<VideoPos> centre(nb);
  std::vector<uint8_t> has_text(nb, 0);
  for (int j = 0; j < L; ++j) {
    SA_REQUIRE(perm[j] >= 0 && perm[j] < L, "sa_local_window_bitmap_perm: perm[%d]=%d outside [0, %d)", j, perm[j], L);
    if (perm[j] < text_len) has_text[j / block] = 1;
  }
  for (int b = 0; b < nb; ++b) centre[b] = token_pos(perm[std::min(b * block + block / 2, L - 1)], text_len, Hp, Wp);
  for (int qb = 0; qb < nb; ++qb) {
    for (int kb = 0; kb < nb; ++kb) {
      const VideoPos& pq = centre[qb];
      const VideoPos& pk = centre[kb];
      const bool win = pq.video && pk.video && iabs(pq.t - pk.t) <= dt && iabs(pq.h - pk.h) <= dh &&
                       iabs(pq.w - pk.w) <= dw;
      bitmap[(int64_t)qb * nb + kb] = (win || has_text[qb] || has_text[kb]) ? 1 : 0;
    }
  }
  return sa::ok();
}

// ---------------------------------------------------------------------------------------
// Sliding-tile attention (SildingTileAttention.py:18-143): the tile-major token order and
// the token-level 3-D tile window, expressed as 64x64 block lists with bitmasks for the
// blocks a tile boundary cuts through.
namespace {

struct StaGeom {
  int text_len, T, Hp, Wp;
  int tt, th, tw;  // tile size
  int kt, kh, kw;  // kernel size in tiles
  int nt, nh, nw;  // tiles per axis
};

// Tile coordinates of a token of the tile-major layout (SildingTileAttention.py:47-54).
inline void sta_tile(const StaGeom& g, int idx, int& t, int& h, int& w) {
  const int tile = (idx - g.text_len) / (g.tt * g.th * g.tw);
  t = tile / (g.nh * g.nw);
  h = (tile % (g.nh * g.nw)) / g.nw;
  w = tile % g.nw;
}

inline int clampi(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }

// sta_mask_3d of SildingTileAttention.py:67-84 for (query, key) tokens of the tile-major
// layout: video pairs inside the clamped 3-D tile window, video->text, text->all.
inline bool sta_allowed(const StaGeom& g, int q, int k) {
  if (q < g.text_len) return true;
  if (k < g.text_len) return true;
  int qt, qh, qw, kt, kh, kw;
  sta_tile(g, q, qt, qh, qw);
  sta_tile(g, k, kt, kh, kw);
  const int ct = clampi(qt, g.kt / 2, (g.nt - 1) - g.kt / 2);
  const int ch = clampi(qh, g.kh / 2, (g.nh - 1) - g.kh / 2);
  const int cw = clampi(qw, g.kw / 2, (g.nw - 1) - g.kw / 2);
  return iabs(ct - kt) <= g.kt / 2 && iabs(ch - kh) <= g.kh / 2 && iabs(cw - kw) <= g.kw / 2;
}

int sta_geom(int text_len, int T, int Hp, int Wp, const int tile[3], const int kernel[3], StaGeom& g) {
  SA_REQUIRE(tile && kernel, "sta: null tile/kernel");
  SA_REQUIRE(text_len >= 0 && T > 0 && Hp > 0 && Wp > 0, "sta: bad geometry");
  SA_REQUIRE(tile[0] > 0 && tile[1] > 0 && tile[2] > 0 && T % tile[0] == 0 && Hp % tile[1] == 0 && Wp % tile[2] == 0,
             "sta: tile (%d,%d,%d) must divide the grid (%d,%d,%d)", tile[0], tile[1], tile[2], T, Hp, Wp);
  SA_REQUIRE(kernel[0] > 0 && kernel[1] > 0 && kernel[2] > 0, "sta: bad kernel");
  g = StaGeom{text_len, T, Hp, Wp, tile[0], tile[1], tile[2], kernel[0], kernel[1], kernel[2],
              T / tile[0], Hp / tile[1], Wp / tile[2]};
  return SA_OK;
}

}  // namespace

extern "C" int sa_sta_permutation(int text_len, int T, int Hp, int Wp, const int tile[3], int32_t* perm) {
  StaGeom g;
  int rc = sta_geom(text_len, T, Hp, Wp, tile, tile, g);
  if (rc) return rc;
  SA_REQUIRE(perm, "sa_sta_permutation: null perm");
  for (int j = 0; j < text_len; ++j) perm[j] = j;
  // "(nt tp nh hp nw wp) -> (nt nh nw tp hp wp)" (SildingTileAttention.py:129-131)
  int j = text_len;
  for (int a = 0; a < g.nt; ++a)
    for (int b = 0; b < g.nh; ++b)
      for (int c = 0; c < g.nw; ++c)
        for (int x = 0; x < g.tt; ++x)
          for (int y = 0; y < g.th; ++y)
            for (int z = 0; z < g.tw; ++z)
              perm[j++] = text_len + ((a * g.tt + x) * Hp + (b * g.th + y)) * Wp + (c * g.tw + z);
  return sa::ok();
}

extern "C" int sa_sta_block_masks(int text_len, int T, int Hp, int Wp, const int tile[3], const int kernel[3],
                                  int32_t* kv_idx, int32_t* kv_cnt, int32_t* kv_slot, uint64_t* masks,
                                  int* n_slots) {
  StaGeom g;
  int rc = sta_geom(text_len, T, Hp, Wp, tile, kernel, g);
  if (rc) return rc;
  SA_REQUIRE(n_slots, "sa_sta_block_masks: null n_slots");
  const int B = 64;
  const int L = text_len + T * Hp * Wp;
  const int nb = sa::cdiv(L, B);
  const bool fill = kv_idx != nullptr;
  SA_REQUIRE(!fill || (kv_cnt && kv_slot), "sa_sta_block_masks: kv_idx without kv_cnt/kv_slot");
  // Tile of every token (-1 for text) and the tile-pair window table: a pair check is then
  // two loads; text rows/columns follow the text rules of sta_allowed.
  const int n_tiles = g.nt * g.nh * g.nw;
  std::vector<int> tile_of(L);
  for (int t = 0; t < L; ++t) tile_of[t] = t < text_len ? -1 : (t - text_len) / (g.tt * g.th * g.tw);
  std::vector<uint8_t> allow((size_t)n_tiles * n_tiles);
  for (int a = 0; a < n_tiles; ++a)
    for (int b = 0; b < n_tiles; ++b) {
      const int qa = text_len + a * g.tt * g.th * g.tw, kb = text_len + b * g.tt * g.th * g.tw;
      allow[(size_t)a * n_tiles + b] = sta_allowed(g, qa, kb) ? 1 : 0;
    }
  int slots = 0;
  uint64_t rows[64];
  for (int qb = 0; qb < nb; ++qb) {
    int cnt = 0;
    for (int kb = 0; kb < nb; ++kb) {
      int any = 0, all = 1;
      const int nk = std::min(B, L - kb * B);
      const uint64_t want = nk == 64 ? ~0ull : ((1ull << nk) - 1);
      for (int r = 0; r < B; ++r) {
        const int q = qb * B + r;
        uint64_t bits = 0;
        if (q < L) {
          const int tq = tile_of[q];
          if (tq < 0) {
            bits = want;  // text query: attends everything
          } else {
            const uint8_t* row = allow.data() + (size_t)tq * n_tiles;
            for (int c = 0; c < nk; ++c) {
              const int tk = tile_of[kb * B + c];
              if (tk < 0 || row[tk]) bits |= 1ull << c;  // video -> text always allowed
            }
          }
        }
        rows[r] = bits;
        any |= bits != 0;
        if (q < L && bits != want) all = 0;
      }
      if (!any) continue;
      if (fill) {
        kv_idx[(int64_t)qb * nb + cnt] = kb;
        kv_slot[(int64_t)qb * nb + cnt] = all ? -1 : slots;
        if (!all && masks) std::memcpy(masks + (int64_t)slots * 64, rows, sizeof(rows));
      }
      if (!all) ++slots;
      ++cnt;
    }
    if (fill) kv_cnt[qb] = cnt;
  }
  *n_slots = slots;
  return sa::ok();
}

// Host mask pipeline: k-hop neighbourhoods, Hilbert order, CSR live-tile lists.
//
// The reference does this at trace time in numpy/scipy (patch.py:208-219): `adj ** k` as a
// sparse matrix power (35 s for the 32-hop r6 mask, docs/results/attn_bwd/...:3), hilbert_order
// (pallas_attn.py:71-82) and build_tile_mask (pallas_attn.py:85-109). Here each stage is a
// multi-threaded pass over CSR rows: a bounded breadth-first search per node for the k-hop
// mask, and a per-row-block merge for the tile list.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <functional>
#include <queue>
#include <thread>
#include <vector>

#include "fwn_attn.h"
#include "fwn_internal.h"

namespace {

int worker_count() {
  unsigned hw = std::thread::hardware_concurrency();
  if (hw == 0) hw = 4;
  return (int)std::min<unsigned>(hw, 16);
}

// Runs fn(begin, end) over [0, n) split into chunks handed out dynamically to the workers.
template <typename Fn>
void parallel_for(int64_t n, int64_t grain, Fn fn) {
  int workers = worker_count();
  if (n <= grain || workers <= 1) {
    fn((int64_t)0, n);
    return;
  }
  std::atomic<int64_t> next(0);
  std::vector<std::thread> pool;
  for (int w = 0; w < workers; ++w) {
    pool.emplace_back([&]() {
      for (;;) {
        int64_t b = next.fetch_add(grain);
        if (b >= n) break;
        fn(b, std::min(n, b + grain));
      }
    });
  }
  for (auto& t : pool) t.join();
}

// Breadth-first ball of radius k around src; `stamp` marks visited nodes with `mark`.
void bfs_ball(int32_t src, int32_t k, const int64_t* adj_ptr, const int32_t* adj_idx,
              std::vector<int32_t>& stamp, int32_t mark, std::vector<int32_t>& ball) {
  ball.clear();
  ball.push_back(src);
  stamp[src] = mark;
  size_t lo = 0;
  for (int32_t hop = 0; hop < k; ++hop) {
    size_t hi = ball.size();
    if (lo == hi) break;
    for (size_t f = lo; f < hi; ++f) {
      int32_t u = ball[f];
      for (int64_t e = adj_ptr[u]; e < adj_ptr[u + 1]; ++e) {
        int32_t w = adj_idx[e];
        if (stamp[w] != mark) {
          stamp[w] = mark;
          ball.push_back(w);
        }
      }
    }
    lo = hi;
  }
}

bool check_adjacency(int32_t n, const int64_t* adj_ptr, const int32_t* adj_idx) {
  if (n <= 0 || !adj_ptr || (adj_ptr[n] > 0 && !adj_idx)) return false;
  if (adj_ptr[0] != 0) return false;
  for (int32_t i = 0; i < n; ++i)
    if (adj_ptr[i + 1] < adj_ptr[i]) return false;
  for (int64_t e = 0; e < adj_ptr[n]; ++e)
    if (adj_idx[e] < 0 || adj_idx[e] >= n) return false;
  return true;
}

// Skilling's transpose algorithm for the 3-D Hilbert index ("Programming the Hilbert curve",
// AIP Conf. Proc. 707, 2004), interleaved most-significant bit first with axis 0 leading each
// triple, as pallas_attn._hilbert3 (pallas_attn.py:41-68).
int64_t hilbert3(int64_t x0, int64_t x1, int64_t x2, int bits) {
  int64_t x[3] = {x0, x1, x2};
  const int64_t top = (int64_t)1 << (bits - 1);
  for (int64_t q = top; q > 1; q >>= 1) {
    const int64_t low = q - 1;
    for (int i = 0; i < 3; ++i) {
      if (x[i] & q) {
        x[0] ^= low;
      } else {
        int64_t t = (x[0] ^ x[i]) & low;
        x[0] ^= t;
        x[i] ^= t;
      }
    }
  }
  x[1] ^= x[0];
  x[2] ^= x[1];
  int64_t flip = 0;
  for (int64_t q = top; q > 1; q >>= 1)
    if (x[2] & q) flip ^= q - 1;
  for (int i = 0; i < 3; ++i) x[i] ^= flip;
  int64_t code = 0;
  for (int b = bits - 1; b >= 0; --b)
    for (int i = 0; i < 3; ++i) code = (code << 1) | ((x[i] >> b) & 1);
  return code;
}

struct Csr {
  int32_t n_rows, n_cols;
  const int64_t* row_ptr;
  const int32_t* idx;
  const int64_t* perm;      // permuted row i is original row perm[i]
  std::vector<int32_t> inv;  // original column c is permuted column inv[c]

  int64_t orig_row(int32_t r) const { return perm ? perm[r] : r; }
  int32_t col(int32_t c) const { return perm ? inv[c] : c; }
};

int make_csr(Csr& m, int32_t n_rows, int32_t n_cols, const int64_t* row_ptr, const int32_t* idx,
             const int64_t* perm) {
  if (n_rows <= 0 || n_cols <= 0 || !row_ptr) return fwn::fail(FWN_ERR_INVALID_ARG, "empty or null mask");
  if (row_ptr[0] != 0) return fwn::fail(FWN_ERR_INVALID_ARG, "row_ptr[0] != 0");
  for (int32_t i = 0; i < n_rows; ++i)
    if (row_ptr[i + 1] < row_ptr[i]) return fwn::fail(FWN_ERR_INVALID_ARG, "row_ptr not monotone");
  if (row_ptr[n_rows] > 0 && !idx) return fwn::fail(FWN_ERR_INVALID_ARG, "null column indices");
  for (int64_t e = 0; e < row_ptr[n_rows]; ++e)
    if (idx[e] < 0 || idx[e] >= n_cols) return fwn::fail(FWN_ERR_INVALID_ARG, "column index out of range");
  m.n_rows = n_rows;
  m.n_cols = n_cols;
  m.row_ptr = row_ptr;
  m.idx = idx;
  m.perm = perm;
  if (perm) {
    if (n_rows != n_cols) return fwn::fail(FWN_ERR_INVALID_ARG, "perm needs a square mask");
    m.inv.assign(n_cols, -1);
    for (int32_t i = 0; i < n_rows; ++i) {
      if (perm[i] < 0 || perm[i] >= n_rows || m.inv[perm[i]] != -1)
        return fwn::fail(FWN_ERR_INVALID_ARG, "perm is not a permutation");
      m.inv[perm[i]] = i;
    }
  }
  return FWN_OK;
}

// Sorted distinct column blocks of row block qb.
void block_columns(const Csr& m, int32_t qb, std::vector<int32_t>& seen, std::vector<int32_t>& out) {
  out.clear();
  int32_t r0 = qb * FWN_BLOCK, r1 = std::min(m.n_rows, r0 + FWN_BLOCK);
  for (int32_t r = r0; r < r1; ++r) {
    int64_t o = m.orig_row(r);
    for (int64_t e = m.row_ptr[o]; e < m.row_ptr[o + 1]; ++e) {
      int32_t kb = m.col(m.idx[e]) / FWN_BLOCK;
      if (seen[kb] != qb) {
        seen[kb] = qb;
        out.push_back(kb);
      }
    }
  }
  std::sort(out.begin(), out.end());
}

}  // namespace

extern "C" {

int fwn_khop_count(int32_t n, const int64_t* adj_ptr, const int32_t* adj_idx, int32_t k,
                   int64_t* row_ptr) {
  fwn::clear_error();
  if (k < 0 || !row_ptr || !check_adjacency(n, adj_ptr, adj_idx))
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_khop_count: invalid adjacency, k or output");
  std::vector<int64_t> size(n);
  parallel_for(n, 256, [&](int64_t b, int64_t e) {
    std::vector<int32_t> stamp(n, -1), ball;
    for (int64_t s = b; s < e; ++s) {
      bfs_ball((int32_t)s, k, adj_ptr, adj_idx, stamp, (int32_t)s, ball);
      size[s] = (int64_t)ball.size();
    }
  });
  row_ptr[0] = 0;
  for (int32_t i = 0; i < n; ++i) row_ptr[i + 1] = row_ptr[i] + size[i];
  return FWN_OK;
}

int fwn_khop_fill(int32_t n, const int64_t* adj_ptr, const int32_t* adj_idx, int32_t k,
                  const int64_t* row_ptr, int32_t* idx) {
  fwn::clear_error();
  if (k < 0 || !row_ptr || !idx || !check_adjacency(n, adj_ptr, adj_idx))
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_khop_fill: invalid adjacency, k or output");
  std::atomic<bool> bad(false);
  parallel_for(n, 256, [&](int64_t b, int64_t e) {
    std::vector<int32_t> stamp(n, -1), ball;
    for (int64_t s = b; s < e; ++s) {
      bfs_ball((int32_t)s, k, adj_ptr, adj_idx, stamp, (int32_t)s, ball);
      if ((int64_t)ball.size() != row_ptr[s + 1] - row_ptr[s]) {
        bad = true;
        return;
      }
      std::sort(ball.begin(), ball.end());
      std::memcpy(idx + row_ptr[s], ball.data(), ball.size() * sizeof(int32_t));
    }
  });
  if (bad) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_khop_fill: row_ptr does not match the k-hop counts");
  return FWN_OK;
}

int fwn_hilbert_order(int64_t n, const double* lat_deg, const double* lon_deg, int32_t bits,
                      int64_t* perm) {
  fwn::clear_error();
  if (n <= 0 || !lat_deg || !lon_deg || !perm || bits < 1 || bits > 20)
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_hilbert_order: invalid arguments");
  const double deg = M_PI / 180.0;
  const double top = (double)((1 << bits) - 1);
  std::vector<int64_t> code(n);
  parallel_for(n, 4096, [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) {
      double la = lat_deg[i] * deg, lo = lon_deg[i] * deg;
      double xyz[3] = {std::cos(la) * std::cos(lo), std::cos(la) * std::sin(lo), std::sin(la)};
      bool finite = std::isfinite(xyz[0]) && std::isfinite(xyz[1]) && std::isfinite(xyz[2]);
      if (!finite) {
        code[i] = INT64_MAX;
        continue;
      }
      int64_t q[3];
      for (int a = 0; a < 3; ++a) {
        double v = std::nearbyint((xyz[a] + 1.0) / 2.0 * top);  // round half to even, as numpy
        q[a] = (int64_t)std::min(std::max(v, 0.0), top);
      }
      code[i] = hilbert3(q[0], q[1], q[2], bits);
    }
  });
  for (int64_t i = 0; i < n; ++i) perm[i] = i;
  std::stable_sort(perm, perm + n, [&](int64_t a, int64_t b) { return code[a] < code[b]; });
  return FWN_OK;
}

int fwn_tiles_count(int32_t n_rows, int32_t n_cols, const int64_t* row_ptr, const int32_t* idx,
                    const int64_t* perm, int32_t* tile_ptr) {
  fwn::clear_error();
  Csr m;
  if (int rc = make_csr(m, n_rows, n_cols, row_ptr, idx, perm)) return rc;
  if (!tile_ptr) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_count: null tile_ptr");
  const int32_t n_qb = (n_rows + FWN_BLOCK - 1) / FWN_BLOCK;
  const int32_t n_kb = (n_cols + FWN_BLOCK - 1) / FWN_BLOCK;
  std::vector<int64_t> count(n_qb);
  parallel_for(n_qb, 4, [&](int64_t b, int64_t e) {
    std::vector<int32_t> seen(n_kb, -1), cols;
    for (int64_t qb = b; qb < e; ++qb) {
      block_columns(m, (int32_t)qb, seen, cols);
      count[qb] = (int64_t)cols.size();
    }
  });
  int64_t total = 0;
  tile_ptr[0] = 0;
  for (int32_t qb = 0; qb < n_qb; ++qb) {
    total += count[qb];
    if (total > INT32_MAX) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_count: too many tiles");
    tile_ptr[qb + 1] = (int32_t)total;
  }
  return FWN_OK;
}

int fwn_tiles_fill(int32_t n_rows, int32_t n_cols, const int64_t* row_ptr, const int32_t* idx,
                   const int64_t* perm, const int32_t* tile_ptr, int32_t* tile_col,
                   uint32_t* tile_bits) {
  fwn::clear_error();
  Csr m;
  if (int rc = make_csr(m, n_rows, n_cols, row_ptr, idx, perm)) return rc;
  const int32_t n_qb = (n_rows + FWN_BLOCK - 1) / FWN_BLOCK;
  // A mask without a valid element has no tiles: the column and bit arrays are then empty and may
  // be null.
  if (!tile_ptr || ((!tile_col || !tile_bits) && tile_ptr[n_qb] > 0))
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_fill: null output");
  const int32_t n_kb = (n_cols + FWN_BLOCK - 1) / FWN_BLOCK;
  const int64_t words = FWN_BLOCK * (FWN_BLOCK / 32);
  std::atomic<bool> bad(false);
  parallel_for(n_qb, 4, [&](int64_t b, int64_t e) {
    std::vector<int32_t> seen(n_kb, -1), local(n_kb, -1), cols;
    for (int64_t qb = b; qb < e; ++qb) {
      block_columns(m, (int32_t)qb, seen, cols);
      const int64_t t0 = tile_ptr[qb];
      if ((int64_t)cols.size() != tile_ptr[qb + 1] - t0) {
        bad = true;
        return;
      }
      for (size_t c = 0; c < cols.size(); ++c) {
        tile_col[t0 + c] = cols[c];
        local[cols[c]] = (int32_t)c;
      }
      std::memset(tile_bits + t0 * words, 0, cols.size() * words * sizeof(uint32_t));
      int32_t r0 = (int32_t)qb * FWN_BLOCK, r1 = std::min(n_rows, r0 + FWN_BLOCK);
      for (int32_t r = r0; r < r1; ++r) {
        int64_t o = m.orig_row(r);
        for (int64_t en = m.row_ptr[o]; en < m.row_ptr[o + 1]; ++en) {
          int32_t j = m.col(m.idx[en]);
          int64_t t = t0 + local[j / FWN_BLOCK];
          int32_t within = j % FWN_BLOCK;
          tile_bits[t * words + (r - r0) * (FWN_BLOCK / 32) + within / 32] |= 1u << (within % 32);
        }
      }
    }
  });
  if (bad) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_fill: tile_ptr does not match the mask");
  return FWN_OK;
}

int fwn_tiles_prepare(int32_t n_blocks, int32_t n_tiles, int32_t n_cols, const int32_t* tile_ptr,
                      const int32_t* tile_col, const uint32_t* tile_bits, uint64_t* lanes,
                      uint32_t* groups, uint32_t* halves) {
  fwn::clear_error();
  if (n_blocks <= 0 || n_tiles < 0 || n_cols <= 0 || !tile_ptr || (n_tiles > 0 && (!tile_col || !tile_bits)) ||
      (n_tiles > 0 && (!lanes || !groups)))
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_prepare: null or empty argument");
  if (int rc = fwn::check_tile_list(n_blocks, n_tiles, n_cols, tile_ptr, tile_col)) return rc;
  const int32_t words = FWN_BLOCK / 32;
  const int32_t tail = n_cols % FWN_BLOCK;  // valid columns in the last column block (0 = all)
  const int32_t last_kb = (n_cols - 1) / FWN_BLOCK;
  std::atomic<bool> bad(false);
  parallel_for(n_tiles, 64, [&](int64_t b, int64_t e) {
    for (int64_t t = b; t < e; ++t) {
      const uint32_t* bits = tile_bits + t * (int64_t)FWN_BLOCK * words;
      if (tile_col[t] == last_kb && tail) {
        for (int32_t r = 0; r < FWN_BLOCK; ++r)
          for (int32_t j = tail; j < FWN_BLOCK; ++j)
            if ((bits[r * words + j / 32] >> (j % 32)) & 1u) bad = true;
      }
      uint32_t f = 0, hv = 0;
      for (int32_t w = 0; w < FWN_WAVES; ++w) {
        for (int32_t x = 0; x < words; ++x) {
          bool any = false, all = true;
          uint32_t lo = 0, hi = 0;
          for (int32_t r = 32 * w; r < 32 * w + 32; ++r) {
            any = any || bits[r * words + x] != 0u;
            all = all && bits[r * words + x] == 0xffffffffu;
            lo |= bits[r * words + x] & 0xffffu;
            hi |= bits[r * words + x] >> 16;
          }
          if (any) f |= 1u << (4 * w + x);
          if (all) f |= 1u << (16 + 4 * w + x);
          if (lo) hv |= 1u << (8 * w + 2 * x);
          if (hi) hv |= 1u << (8 * w + 2 * x + 1);
        }
        for (int32_t lane = 0; lane < 64; ++lane) {
          const int32_t row = 32 * w + (lane & 31);
          uint64_t word = 0;
          for (int32_t el = 0; el < 64; ++el) {
            const int32_t key = fwn::element_col(el >> 4, el & 15, lane >> 5);
            word |= (uint64_t)((bits[row * words + key / 32] >> (key % 32)) & 1u) << el;
          }
          lanes[t * FWN_LANE_WORDS + w * 64 + lane] = word;
        }
      }
      groups[t] = f;
      if (halves) halves[t] = hv;
    }
  });
  if (bad) return fwn::fail(FWN_ERR_TILES, "fwn_tiles_prepare: a tile has bits set beyond n_cols");
  return FWN_OK;
}

int fwn_tiles_ds_map(int32_t n_blocks, const int32_t* tile_ptr, const int32_t* tile_col,
                     const uint32_t* tile_bits, const int32_t* tile_ptr_t, const int32_t* tile_col_t,
                     const uint32_t* tile_bits_t, int32_t unit_keys, int32_t* ubase, int32_t* tmap,
                     int64_t* n_units) {
  fwn::clear_error();
  if (n_blocks <= 0 || !tile_ptr || !tile_ptr_t || !n_units)
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_ds_map: null or empty argument");
  if (unit_keys != 16 && unit_keys != 32)
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_ds_map: unit_keys %d (16 or 32)", unit_keys);
  const int32_t n_tiles = tile_ptr[n_blocks], n_tiles_t = tile_ptr_t[n_blocks];
  if (n_tiles > 0 && (!tile_col || !tile_bits || !ubase))
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_ds_map: null forward arrays");
  if (n_tiles_t > 0 && (!tile_col_t || !tile_bits_t || !tmap))
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_ds_map: null transposed arrays");
  const int32_t n_cols = n_blocks * FWN_BLOCK;
  if (int rc = fwn::check_tile_list(n_blocks, n_tiles, n_cols, tile_ptr, tile_col)) return rc;
  if (int rc = fwn::check_tile_list(n_blocks, n_tiles_t, n_cols, tile_ptr_t, tile_col_t)) return rc;
  if (n_tiles != n_tiles_t)
    return fwn::fail(FWN_ERR_TILES, "fwn_tiles_ds_map: %d forward tiles but %d transposed ones", n_tiles, n_tiles_t);
  constexpr int32_t words = FWN_BLOCK / 32;
  constexpr int64_t tile_words = (int64_t)FWN_BLOCK * words;
  // Unit bits of each forward tile, as fwn_tiles_prepare computes them: the half bits (bit
  // 8r + 2c + h: rows 32r.., columns 32c + 16h ..) for 16-key units, the group bits (bit 4r + c)
  // for 32-key units; and the exclusive prefix of their counts.
  std::vector<uint32_t> halves(n_tiles);
  parallel_for(n_tiles, 256, [&](int64_t b, int64_t e) {
    for (int64_t t = b; t < e; ++t) {
      const uint32_t* bits = tile_bits + t * tile_words;
      uint32_t hv = 0;
      for (int32_t r = 0; r < FWN_BLOCK; ++r)
        for (int32_t x = 0; x < words; ++x) {
          const uint32_t wd = bits[r * words + x];
          if (unit_keys == 32) {
            if (wd) hv |= 1u << (4 * (r / 32) + x);
            continue;
          }
          if (wd & 0xffffu) hv |= 1u << (8 * (r / 32) + 2 * x);
          if (wd >> 16) hv |= 1u << (8 * (r / 32) + 2 * x + 1);
        }
      halves[t] = hv;
    }
  });
  int64_t total = 0;
  for (int32_t t = 0; t < n_tiles; ++t) {
    ubase[t] = (int32_t)total;
    total += __builtin_popcount(halves[t]);
    if (total > INT32_MAX) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_ds_map: more than 2^31 units");
  }
  // Each transposed tile (row block kb, column block qb) must be forward tile (qb, kb) with its
  // bits transposed.
  std::atomic<int64_t> bad(-1);
  parallel_for(n_tiles_t, 64, [&](int64_t b, int64_t e) {
    std::vector<uint32_t> tr(tile_words);
    int32_t kb = (int32_t)(std::upper_bound(tile_ptr_t, tile_ptr_t + n_blocks + 1, (int32_t)b) - tile_ptr_t) - 1;
    for (int64_t t = b; t < e; ++t) {
      while (tile_ptr_t[kb + 1] <= t) ++kb;
      const int32_t qb = tile_col_t[t];
      const int32_t* lo = tile_col + tile_ptr[qb];
      const int32_t* hi = tile_col + tile_ptr[qb + 1];
      const int32_t* it = std::lower_bound(lo, hi, kb);
      if (it == hi || *it != kb) {
        bad = t;
        return;
      }
      const int64_t tf = it - tile_col;
      std::fill(tr.begin(), tr.end(), 0u);
      const uint32_t* fb = tile_bits + tf * tile_words;
      for (int32_t r = 0; r < FWN_BLOCK; ++r)
        for (int32_t x = 0; x < words; ++x)
          for (uint32_t wd = fb[r * words + x]; wd; wd &= wd - 1) {
            const int32_t c = 32 * x + __builtin_ctz(wd);
            tr[c * words + r / 32] |= 1u << (r % 32);
          }
      if (std::memcmp(tr.data(), tile_bits_t + t * tile_words, tile_words * sizeof(uint32_t)) != 0) {
        bad = t;
        return;
      }
      tmap[2 * t] = ubase[tf];
      tmap[2 * t + 1] = (int32_t)halves[tf];
    }
  });
  if (bad.load() >= 0)
    return fwn::fail(FWN_ERR_TILES, "fwn_tiles_ds_map: the second list is not the transpose of the first (tile %lld)",
                     (long long)bad.load());
  *n_units = total;
  return FWN_OK;
}

int fwn_tiles_schedule_count(int32_t n_blocks, const int32_t* tile_ptr, int32_t max_item_tiles,
                             int32_t* n_items, int32_t* n_parts, int32_t* n_split) {
  fwn::clear_error();
  if (n_blocks <= 0 || !tile_ptr || !n_items || !n_parts || !n_split)
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_schedule_count: null or empty argument");
  const int64_t chunk = max_item_tiles > 0 ? max_item_tiles : FWN_ITEM_TILES;
  int64_t items = 0, parts = 0, split = 0;
  for (int32_t b = 0; b < n_blocks; ++b) {
    const int64_t count = (int64_t)tile_ptr[b + 1] - tile_ptr[b];
    if (count < 0) return fwn::fail(FWN_ERR_TILES, "fwn_tiles_schedule_count: tile_ptr decreases at block %d", b);
    const int64_t p = count > chunk ? (count + chunk - 1) / chunk : 1;
    items += p;
    if (p > 1) {
      parts += p;
      ++split;
    }
  }
  if (items > INT32_MAX) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_schedule_count: too many items");
  *n_items = (int32_t)items;
  *n_parts = (int32_t)parts;
  *n_split = (int32_t)split;
  return FWN_OK;
}

int fwn_tiles_schedule_fill(int32_t n_blocks, const int32_t* tile_ptr, int32_t max_item_tiles,
                            fwn_item* items, int32_t* split) {
  fwn::clear_error();
  int32_t n_items = 0, n_parts = 0, n_split = 0;
  if (int rc = fwn_tiles_schedule_count(n_blocks, tile_ptr, max_item_tiles, &n_items, &n_parts, &n_split))
    return rc;
  if (!items || (n_split > 0 && !split))
    return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_schedule_fill: null output");
  const int64_t chunk = max_item_tiles > 0 ? max_item_tiles : FWN_ITEM_TILES;
  int32_t it = 0, part = 0, sp = 0;
  for (int32_t b = 0; b < n_blocks; ++b) {
    const int32_t t0 = tile_ptr[b], count = tile_ptr[b + 1] - t0;
    const int32_t p = count > chunk ? (int32_t)((count + chunk - 1) / chunk) : 1;
    if (p == 1) {
      items[it++] = fwn_item{b, t0, t0 + count, -1};
      continue;
    }
    split[3 * sp] = b;
    split[3 * sp + 1] = part;
    split[3 * sp + 2] = p;
    ++sp;
    // Near-equal runs: the first count % p runs get one tile more.
    int32_t t = t0;
    for (int32_t c = 0; c < p; ++c) {
      const int32_t len = count / p + (c < count % p ? 1 : 0);
      items[it++] = fwn_item{b, t, t + len, part++};
      t += len;
    }
  }
  return FWN_OK;
}

}  // extern "C"

namespace {

// The jobs of each XCD for an order table (fwn_tiles_order_count / _fill): job j is item
// j % n_items of pair j / n_items.
// The jobs [b0, b1) of one XCD in launch order: job order, then each window of `window` jobs
// (counted from the range's end, so the last `window` jobs, the launch's last rounds, are one
// full window and the first window takes the remainder) sorted longest first.
void range_order(int64_t b0, int64_t b1, int32_t window, const std::vector<int64_t>& cost, int32_t n_items,
                 std::vector<int64_t>& r) {
  r.clear();
  for (int64_t j = b0; j < b1; ++j) r.push_back(j);
  if (window > 1)
    for (size_t w0 = 0, w1 = r.size() % (size_t)window; w0 < r.size(); w0 = w1, w1 += (size_t)window) {
      if (w1 == w0) continue;
      std::stable_sort(r.begin() + (ptrdiff_t)w0, r.begin() + (ptrdiff_t)w1,
                       [&](int64_t p, int64_t q) { return cost[p % n_items] > cost[q % n_items]; });
    }
}

// When the last of the jobs `r` ends if `slots` slots take them in order, each job going to the
// first free slot and lasting its cost.
int64_t makespan(const std::vector<int64_t>& r, const std::vector<int64_t>& cost, int32_t n_items, int32_t slots) {
  std::priority_queue<int64_t, std::vector<int64_t>, std::greater<int64_t>> free_at;
  for (int32_t s = 0; s < slots; ++s) free_at.push(0);
  int64_t end = 0;
  for (int64_t j : r) {
    const int64_t t = free_at.top() + cost[j % n_items];
    free_at.pop();
    free_at.push(t);
    end = std::max(end, t);
  }
  return end;
}

int order_ranges(int32_t n_items, const fwn_item* items, const int32_t* tile_cost, int32_t item_cost,
                 int32_t pairs, int32_t order, int32_t window, int32_t slots, const char* what,
                 std::vector<std::vector<int64_t>>& xcd) {
  if (n_items <= 0 || !items || pairs <= 0 || item_cost < 0)
    return fwn::fail(FWN_ERR_INVALID_ARG, "%s: null, empty or negative argument", what);
  if (order != FWN_ORDER_ITEMS && order != FWN_ORDER_BALANCED && order != FWN_ORDER_MAKESPAN)
    return fwn::fail(FWN_ERR_INVALID_ARG, "%s: unknown order %d", what, order);
  if (order == FWN_ORDER_MAKESPAN && (slots <= 0 || slots > 65536))
    return fwn::fail(FWN_ERR_INVALID_ARG, "%s: FWN_ORDER_MAKESPAN needs 1 to 65536 slots (got %d)", what, slots);
  const int64_t jobs = (int64_t)n_items * pairs;
  if (jobs > INT32_MAX) return fwn::fail(FWN_ERR_INVALID_ARG, "%s: too many jobs", what);
  std::vector<int64_t> cost((size_t)n_items);
  int64_t per_pair = 0;
  for (int32_t i = 0; i < n_items; ++i) {
    const int64_t len = (int64_t)items[i].t1 - items[i].t0;
    if (len < 0 || items[i].t0 < 0) return fwn::fail(FWN_ERR_TILES, "%s: item %d has no valid tile range", what, i);
    cost[i] = item_cost;
    if (!tile_cost) {
      cost[i] += len;
    } else {
      for (int32_t t = items[i].t0; t < items[i].t1; ++t) {
        if (tile_cost[t] < 0) return fwn::fail(FWN_ERR_INVALID_ARG, "%s: tile %d has a negative cost", what, t);
        cost[i] += tile_cost[t];
      }
    }
    per_pair += cost[i];
  }
  // XCD x takes jobs [bound[x], bound[x + 1]): equal counts as the kernels' own mapping, or, by
  // cost, the jobs whose cost midpoint lies in [x / 8, (x + 1) / 8) of the total (each range
  // then costs its share to within one job).
  int64_t bound[9];
  const int64_t total = per_pair * pairs;
  if (order == FWN_ORDER_ITEMS || total == 0) {
    const int64_t small = jobs / 8, rem = jobs % 8;
    bound[0] = 0;
    for (int x = 0; x < 8; ++x) bound[x + 1] = bound[x] + small + (x < rem ? 1 : 0);
  } else {
    int64_t before = 0;
    int x = 0;
    bound[0] = 0;
    for (int64_t j = 0; j < jobs; ++j) {
      const int64_t c = cost[j % n_items];
      // twice the midpoint, 2 before + c, in eighths of the total: XCD (2 before + c) * 4 / total
      const int64_t xj = std::min<int64_t>(7, (2 * before + c) * 4 / total);
      while (x < xj) bound[++x] = j;
      before += c;
    }
    while (x < 8) bound[++x] = jobs;
  }
  xcd.assign(8, {});
  for (int x = 0; x < 8; ++x) range_order(bound[x], bound[x + 1], window, cost, n_items, xcd[x]);
  if (order == FWN_ORDER_MAKESPAN && total > 0) {
    // From the equal-cost ranges, move one job at a time across a boundary of the XCD that ends
    // last (its first job to the XCD before, or its last to the XCD after), while that lowers
    // the later end of the two.
    int64_t ms[8];
    for (int x = 0; x < 8; ++x) ms[x] = makespan(xcd[x], cost, n_items, slots);
    std::vector<int64_t> ra, rb;
    for (int64_t step = 0; step < 64 * (jobs + 8); ++step) {
      const int x = (int)(std::max_element(ms, ms + 8) - ms);
      int best_side = 0;
      int64_t best = ms[x], best_a = 0, best_b = 0;
      for (int side = -1; side <= 1; side += 2) {
        const int y = x + side;
        if (y < 0 || y > 7 || bound[x + 1] == bound[x]) continue;
        // side -1: job bound[x] moves to XCD x - 1; side +1: job bound[x + 1] - 1 moves to x + 1
        const int64_t nb = side < 0 ? bound[x] + 1 : bound[x + 1] - 1;
        if (side < 0) {
          range_order(nb, bound[x + 1], window, cost, n_items, ra);
          range_order(bound[y], nb, window, cost, n_items, rb);
        } else {
          range_order(bound[x], nb, window, cost, n_items, ra);
          range_order(nb, bound[y + 1], window, cost, n_items, rb);
        }
        const int64_t a = makespan(ra, cost, n_items, slots), b = makespan(rb, cost, n_items, slots);
        if (std::max(a, b) < best) {
          best = std::max(a, b);
          best_side = side;
          best_a = a;
          best_b = b;
        }
      }
      if (best_side == 0) break;
      const int y = x + best_side;
      if (best_side < 0) {
        ++bound[x];
      } else {
        --bound[x + 1];
      }
      range_order(bound[x], bound[x + 1], window, cost, n_items, xcd[x]);
      range_order(bound[y], bound[y + 1], window, cost, n_items, xcd[y]);
      ms[x] = best_a;
      ms[y] = best_b;
    }
  }
  return FWN_OK;
}

int64_t order_entries(const std::vector<std::vector<int64_t>>& xcd) {
  size_t most = 0;
  for (const auto& r : xcd) most = std::max(most, r.size());
  return 8 * (int64_t)most;
}

}  // namespace

extern "C" {

int fwn_tiles_order_count(int32_t n_items, const fwn_item* items, const int32_t* tile_cost, int32_t item_cost,
                          int32_t pairs, int32_t order, int32_t window, int32_t slots, int32_t* n_work) {
  fwn::clear_error();
  if (!n_work) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_order_count: null output");
  std::vector<std::vector<int64_t>> xcd;
  if (int rc = order_ranges(n_items, items, tile_cost, item_cost, pairs, order, window, slots, "fwn_tiles_order_count",
                            xcd))
    return rc;
  const int64_t entries = order_entries(xcd);
  if (entries > INT32_MAX) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_order_count: too many entries");
  *n_work = (int32_t)entries;
  return FWN_OK;
}

int fwn_tiles_order_fill(int32_t n_items, const fwn_item* items, const int32_t* tile_cost, int32_t item_cost,
                         int32_t pairs, int32_t order, int32_t window, int32_t slots, int32_t* work) {
  fwn::clear_error();
  if (!work) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_order_fill: null output");
  std::vector<std::vector<int64_t>> xcd;
  if (int rc = order_ranges(n_items, items, tile_cost, item_cost, pairs, order, window, slots, "fwn_tiles_order_fill",
                            xcd))
    return rc;
  const int64_t entries = order_entries(xcd);
  if (entries > INT32_MAX) return fwn::fail(FWN_ERR_INVALID_ARG, "fwn_tiles_order_fill: too many entries");
  // The k-th job of XCD x goes to workgroup 8 k + x; the rest are padding.
  for (int64_t w = 0; w < entries; ++w) {
    work[2 * w] = -1;
    work[2 * w + 1] = 0;
  }
  for (int x = 0; x < 8; ++x)
    for (size_t k = 0; k < xcd[x].size(); ++k) {
      const int64_t j = xcd[x][k], w = 8 * (int64_t)k + x;
      work[2 * w] = (int32_t)(j / n_items);
      work[2 * w + 1] = (int32_t)(j % n_items);
    }
  return FWN_OK;
}

}  // extern "C"

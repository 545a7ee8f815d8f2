// market.hip -- MI355X (gfx950) VecMarket order-matching engine behind the C ABI
// declared in include/astra_market.h.
//
// Semantics follow the reference kernels of nlyu1/astra-cuda
// src/order_matching/market.cu (add_orders_kernel :17-100, match_orders_kernel
// :102-278, get_bbo_kernel :280-320, update_last_prices_kernel :767-786) bit for
// bit, including what ring-slot reuse does to the level lists (a reused slot is
// never unlinked, so stale heads, cut chains, self links and zero/negative-size
// fills happen exactly as in the reference). The data layout and the kernels are
// this engine's own:
//
//  * One lane per market. A market's matching is a serial dependency chain
//    (each fill decides the next pair of heads), so the 64 lanes of a wavefront
//    carry 64 independent markets and the memory system sees M independent
//    chains at once.
//  * Per market and side, the occupancy of the L price levels is a bitmask of
//    W = ceil(L/64) 64-bit words kept in registers during a call; bit p is set
//    exactly when the level's head is not NULL. Best bid / best ask are
//    count-leading/trailing-zeros over the mask, replacing the reference's
//    O(L) rescans. The masks live in HBM as structure-of-arrays
//    mask[side][word][market], so their loads and stores are fully coalesced.
//  * Level lists are packed: level p of market m is 8 bytes
//    {bid_head, bid_tail, ask_head, ask_tail} as uint16 (NULL = 0xFFFF), so one
//    32-bit access reads or writes a side's head and tail together and the
//    levels around the mid share a few 128-byte lines.
//  * An order slot is one 16-byte record {size, customer, tid, price | next<<16},
//    read with a single 128-bit load. order_is_bid is not stored: nothing in the
//    reference ever reads it (written at market.cu:54,83 only).
//  * Portfolio updates are fire-and-forget atomic adds (no return value), so
//    they stay off the matching chain. int32 wrap-around is the same as the
//    reference's plain += / -=.
//
// Behaviour the reference leaves undefined (out-of-bounds indexing) is defined
// here and in the CPU oracle in the same way: negative prices are not inserted,
// negative customer ids do not touch portfolios. Every slot index read from the
// book is bounds-checked before it is dereferenced.
//
// Every kernel body is a __host__ __device__ function behind a thin __global__
// wrapper. Built with -DASTRA_HOST_EMULATION (host-only compile), the same
// bodies run in plain loops over host memory behind the same C ABI; the tests
// use that build to check the logic and its bounds on the CPU.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#define ASTRA_SRC_NAME "market.hip"
#include "runtime.h"
#include "game_move.h"

using namespace astra_rt;

namespace {

constexpr uint32_t kNull16 = 0xFFFFu;
// Bit 15 of a head slot in the tob word: that head order's size is in the
// workspace's head-size cache (slots are below 0x8000 since O <= 32768; NULL is
// 0xFFFF and carries no flag).
constexpr uint32_t kSizeKnown = 0x8000u;
constexpr int kFillThreads = 256;

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline int mask_words_for(int32_t L) {
  const int w = (L + 63) / 64;
  if (w <= 1) return 1;
  if (w <= 2) return 2;
  if (w <= 4) return 4;
  if (w <= 8) return 8;
  return 16;
}

// Control words at the start of the workspace (int32): the TID counter of a
// market with no markets (market.h:338; with markets it lives in Book::tids),
// and the number of helper wavefronts that gave up waiting (a diagnostic count).
constexpr int kCtlTid = 0;
constexpr int kCtlHelperExits = 1;
constexpr size_t kCtlBytes = 256;

// Byte offsets of the book arrays inside the workspace.
struct Layout {
  int W;
  size_t ctl, masks, next_slot, tids, bbo, tob, hsz, levels, records, portfolios, total;
};

Layout make_layout(int64_t M, int64_t L, int64_t O, int64_t C) {
  Layout l;
  l.W = mask_words_for((int32_t)L);
  size_t off = 0;
  l.ctl = off;
  off += kCtlBytes;
  l.masks = off;
  off = align_up(off + (size_t)2 * l.W * M * 8, 256);
  l.next_slot = off;
  off = align_up(off + (size_t)M * 4, 256);
  l.tids = off;
  off = align_up(off + (size_t)M * 4, 256);
  l.bbo = off;
  off = align_up(off + (size_t)2 * M * 4, 256);
  l.tob = off;
  off = align_up(off + (size_t)M * 4, 256);
  l.hsz = off;
  off = align_up(off + (size_t)2 * M * 4, 256);
  l.levels = off;
  off = align_up(off + (size_t)M * L * 8, 256);
  l.records = off;
  off = align_up(off + (size_t)M * O * 16, 256);
  l.portfolios = off;
  off = align_up(off + (size_t)M * C * 8, 256);
  l.total = off;
  return l;
}

}  // namespace

struct astra_market {
  int32_t M, L, O, F, C;
  int device;
  int32_t threads_per_block;  // validated, not used for launches
  int32_t flags;
  int block;                  // launch block size of the per-market kernels
  int32_t stage_budget;       // loop passes before a market is staged in LDS (0: never)
  int32_t lds_limit;          // LDS bytes a workgroup may use on the device
  int32_t lds_per_cu;         // LDS bytes of one CU
  int32_t cus;                // CUs of the device
  int32_t per_wave;           // markets per wavefront of the matching kernel (0: default)
  int32_t fill_rows;          // fill rows a lane buffers before writing them (0: by grid)
  int32_t helpers;            // market wavefronts per helper wavefront (0: no helpers)
  int32_t hand_lanes;         // zero-size walks go to the helper when at most this many lanes loop
  int32_t hand_queue;         // no hand-off while this many markets wait for the helper
  int32_t helper_polls;       // idle polls before a helper wavefront gives up
  int32_t scratch_word;       // word of the per-device scratch its allocation-free moves use (-1: none)
  unsigned long long *stats;  // see astra_market_set_stats
  char *ws;
  size_t ws_bytes;
  Layout lay;
};

namespace {

struct Book {
  int32_t *ctl;               // the control words (kCtl*)
  uint64_t *masks;            // [2][W][M]: side 0 = bid, 1 = ask
  int32_t *next_slot;         // [M], in [0, O)
  int32_t *tids;              // [M]: the TID counter (market.h:338), one copy per market
  int32_t *bbo;               // [2][M]: best bid price, best ask price (NULL: empty side)
  uint32_t *tob;              // [M]: head slots of the best levels, bid | ask << 16, each
                              // with kSizeKnown set when its size is in hsz
  int32_t *hsz;               // [2][M]: sizes of those head orders (valid where flagged)
  uint16_t *levels;           // [M][L][4] = {bid_head, bid_tail, ask_head, ask_tail}
  uint4 *records;             // [M][O] = {size, customer, tid, price | next << 16}
  int32_t *portfolios;        // [M][C][2] = {contracts, cash}
  unsigned long long *stats;  // diagnostic counters [11] or nullptr
  int32_t M, L, O, F, C;
};

Book book_of(const astra_market *h) {
  Book b;
  b.ctl = reinterpret_cast<int32_t *>(h->ws + h->lay.ctl);
  b.masks = reinterpret_cast<uint64_t *>(h->ws + h->lay.masks);
  b.next_slot = reinterpret_cast<int32_t *>(h->ws + h->lay.next_slot);
  b.tids = reinterpret_cast<int32_t *>(h->ws + h->lay.tids);
  b.bbo = reinterpret_cast<int32_t *>(h->ws + h->lay.bbo);
  b.tob = reinterpret_cast<uint32_t *>(h->ws + h->lay.tob);
  b.hsz = reinterpret_cast<int32_t *>(h->ws + h->lay.hsz);
  b.levels = reinterpret_cast<uint16_t *>(h->ws + h->lay.levels);
  b.records = reinterpret_cast<uint4 *>(h->ws + h->lay.records);
  b.portfolios = reinterpret_cast<int32_t *>(h->ws + h->lay.portfolios);
  b.stats = h->stats;
  b.M = h->M;
  b.L = h->L;
  b.O = h->O;
  b.F = h->F;
  b.C = h->C;
  return b;
}

// The call's quotes: five [M] columns, or (the game's trading move) the [M,4]
// move rows and the acting player in `game`.
struct QuoteIn {
  const int32_t *bid_px, *bid_sz, *ask_px, *ask_sz, *cust;
  GameMove game;
};

// Fill rows go either to the reference's eight [M,F] arrays or, when `rows` is
// set, to one [M,F,8] int32 array: row (m, k) is 32 contiguous bytes {price,
// size, taker, quoter, is_sell (0/1), quote size, tid, quote tid}.
struct FillOut {
  int32_t *prices, *sizes, *taker, *quoter;
  uint8_t *is_sell_quote;
  int32_t *quote_sizes, *tid, *quote_tid, *counts;
  int32_t *rows;
};

// Per-step outputs of a multi-step call (null when not wanted): every step's
// fill counts ([steps, M]) and every step's GetBBOs ([4, steps, M]: bid price,
// bid size, ask price, ask size). Inside the kernel the pointers are those of
// the current step ([M] each, bbo[j] the j-th field).
struct StepOut {
  int32_t *counts;
  int32_t *bbo[4];
};

// The quotes and per-step outputs of step k of a multi-step call: the [steps, M]
// inputs at row k.
ASTRA_HD void step_views(const QuoteIn &in, const StepOut &so, int64_t M, int32_t steps, int32_t k,
                         QuoteIn &ink, StepOut &sok) {
  const int64_t off = (int64_t)k * M;
  ink = in;
  ink.bid_px = in.bid_px + off;
  ink.bid_sz = in.bid_sz + off;
  ink.ask_px = in.ask_px + off;
  ink.ask_sz = in.ask_sz + off;
  ink.cust = in.cust + off;
  sok.counts = so.counts ? so.counts + off : nullptr;
  for (int j = 0; j < 4; ++j)
    sok.bbo[j] = so.bbo[0] ? so.bbo[0] + ((int64_t)j * steps * M + off) : nullptr;
}

// ---- small device/host helpers ----

ASTRA_HD int clz64(uint64_t x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __clzll(x);
#else
  return x ? __builtin_clzll(x) : 64;
#endif
}

ASTRA_HD int ctz64(uint64_t x) {  // x != 0
#if defined(__HIP_DEVICE_COMPILE__)
  return __ffsll((unsigned long long)x) - 1;
#else
  return __builtin_ctzll(x);
#endif
}

// A market still crossing when at most this many lanes of its wavefront are
// still in their matching loop, and about to walk zero-size orders, is staged
// at once rather than after the pass budget. Not in the game move: at the
// config-5 shape (10,000 envs, 32 per wavefront) it made the move 16% slower.
constexpr int32_t kEarlyStageLanes = 2;

// How many lanes of the wavefront execute this point together (the host build
// runs one market at a time: 1).
ASTRA_HD int32_t lanes_here() {
#if defined(__HIP_DEVICE_COMPILE__)
  return (int32_t)__popcll(__ballot(1));
#else
  return 1;
#endif
}

// Fire-and-forget add with int32 wrap-around.
ASTRA_HD void add_i32(int32_t *p, int32_t v) {
#if defined(__HIP_DEVICE_COMPILE__)
  atomicAdd(p, v);
#else
  *p = (int32_t)((uint32_t)*p + (uint32_t)v);
#endif
}

ASTRA_HD void add_u64(unsigned long long *p, unsigned long long v) {
#if defined(__HIP_DEVICE_COMPILE__)
  atomicAdd(p, v);
#else
  *p += v;
#endif
}

ASTRA_HD int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }

// ---- occupancy-mask helpers (W words, fully unrolled, no dynamic indexing) ----

template <int W>
ASTRA_HD int mask_highest(const uint64_t (&m)[W]) {
  int r = -1;
#pragma unroll
  for (int i = 0; i < W; ++i)
    if (m[i]) r = i * 64 + 63 - clz64(m[i]);
  return r;
}

template <int W>
ASTRA_HD int mask_lowest(const uint64_t (&m)[W], int none) {
  int r = none;
#pragma unroll
  for (int i = W - 1; i >= 0; --i)
    if (m[i]) r = i * 64 + ctz64(m[i]);
  return r;
}

// Bit updates are arithmetic per word (no branch selects the word), so the
// compiler keeps the mask in registers instead of forming an indexed array.
template <int W>
ASTRA_HD void mask_set(uint64_t (&m)[W], int p) {
#pragma unroll
  for (int i = 0; i < W; ++i) m[i] |= (uint64_t)((p >> 6) == i) << (p & 63);
}

template <int W>
ASTRA_HD void mask_clear(uint64_t (&m)[W], int p) {
#pragma unroll
  for (int i = 0; i < W; ++i) m[i] &= ~((uint64_t)((p >> 6) == i) << (p & 63));
}

// Byte offsets of one side's {head, tail} pair within a level: side 0 = bid, 1 = ask.
ASTRA_HD uint32_t level_word(const uint16_t *lv, int32_t price, int side) {
  return *reinterpret_cast<const uint32_t *>(lv + (size_t)price * 4 + 2 * side);
}

// The head slot of level `price` on `side` (the low half of its word).
ASTRA_HD uint32_t level_head(const uint16_t *lv, int32_t price, int side) {
  return lv[(size_t)price * 4 + 2 * side];
}

ASTRA_HD void store_level_word(uint16_t *lv, int32_t price, int side, uint32_t w) {
  *reinterpret_cast<uint32_t *>(lv + (size_t)price * 4 + 2 * side) = w;
}

ASTRA_HD void store_head(uint16_t *lv, int32_t price, int side, uint32_t head) {
  lv[(size_t)price * 4 + 2 * side] = (uint16_t)head;
}

ASTRA_HD uint32_t rec_next(const uint4 &r) { return r.w >> 16; }
ASTRA_HD uint4 with_next(uint4 r, uint32_t next) {
  r.w = (r.w & kNull16) | (next << 16);
  return r;
}

// Rows that a market still owes when its matching loop has reached a state that
// repeats forever; the caller writes them (cooperatively on the GPU).
struct Bulk {
  int64_t base;   // first fill index (m * F + k)
  int32_t count;  // rows to write
  int32_t alt;    // 1: negate size and quote size on every odd row
  int32_t v[8];   // price, size, taker, quoter, is_sell_quote, quote_size, tid, quote_tid
};

// A store into the caller's fill batch through a global-address-space pointer.
// The kernel holds the batch pointers in VGPRs (in_vgpr), where the compiler no
// longer knows they point to global memory; plain stores through them become
// flat stores, which also count against the LDS/scalar counter, so every later
// wait for an LDS access would wait for those stores to reach memory too.
// HIP's vector types assign through a member operator, whose `this` is a
// generic pointer, so their lanes go out as a native vector (2 or 4 lanes) or
// as three 4-byte stores (which the compiler merges into one 12-byte store;
// a 3-lane native vector would be stored as 4 lanes, one too many).
template <class T>
ASTRA_HD void gst(T *p, const T &v) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (std::is_same_v<T, int4> || std::is_same_v<T, uint4>) {
    typedef int32_t v4 __attribute__((ext_vector_type(4)));
    *(__attribute__((address_space(1))) v4 *)p =
        v4{(int32_t)v.x, (int32_t)v.y, (int32_t)v.z, (int32_t)v.w};
  } else if constexpr (std::is_same_v<T, int2> || std::is_same_v<T, uint2>) {
    typedef int32_t v2 __attribute__((ext_vector_type(2)));
    *(__attribute__((address_space(1))) v2 *)p = v2{(int32_t)v.x, (int32_t)v.y};
  } else if constexpr (std::is_same_v<T, int3>) {
    __attribute__((address_space(1))) int32_t *q = (__attribute__((address_space(1))) int32_t *)p;
    q[0] = v.x;
    q[1] = v.y;
    q[2] = v.z;
  } else {
    *(__attribute__((address_space(1))) T *)p = v;
  }
#else
  *p = v;
#endif
}

ASTRA_HD void write_row(int32_t *rows, int64_t fi, const int32_t (&v)[8]) {
  int4 *d = reinterpret_cast<int4 *>(rows + fi * 8);
  gst(d, make_int4(v[0], v[1], v[2], v[3]));
  gst(d + 1, make_int4(v[4], v[5], v[6], v[7]));
}

ASTRA_HD void write_fill(const FillOut &out, int64_t fi, const int32_t (&v)[8]) {
  if (out.rows) {
    write_row(out.rows, fi, v);
    return;
  }
  gst(out.prices + fi, v[0]);
  gst(out.sizes + fi, v[1]);
  gst(out.taker + fi, v[2]);
  gst(out.quoter + fi, v[3]);
  gst(out.is_sell_quote + fi, (uint8_t)v[4]);
  gst(out.quote_sizes + fi, v[5]);
  gst(out.tid + fi, v[6]);
  gst(out.quote_tid + fi, v[7]);
}

// Host build: write the owed rows directly.
inline void write_bulk_host(const FillOut &out, const Bulk &bk) {
  for (int32_t k = 0; k < bk.count; ++k) {
    int32_t v[8];
    for (int i = 0; i < 8; ++i) v[i] = bk.v[i];
    if (bk.alt && (k & 1)) {
      v[1] = (int32_t)(0u - (uint32_t)v[1]);
      v[5] = (int32_t)(0u - (uint32_t)v[5]);
    }
    write_fill(out, bk.base + k, v);
  }
}

// The fill row of one pass (market.cu:172-218): the earlier TID rests (ties go
// to the ask side); price, quote size and quote TID are the resting order's.
ASTRA_HD void make_row(const uint4 &b, const uint4 &a, int32_t qty, int32_t (&row)[8]) {
  const bool bid_quote = (int32_t)b.z < (int32_t)a.z;
  row[0] = (int32_t)((bid_quote ? b.w : a.w) & kNull16);
  row[1] = qty;
  row[2] = (int32_t)(bid_quote ? a.y : b.y);
  row[3] = (int32_t)(bid_quote ? b.y : a.y);
  row[4] = bid_quote ? 0 : 1;
  row[5] = (int32_t)(bid_quote ? b.x : a.x);
  row[6] = (int32_t)(bid_quote ? a.z : b.z);
  row[7] = (int32_t)(bid_quote ? b.z : a.z);
}

// Portfolio update of one fill row (market.cu:221-232): the buyer is the bid
// side's customer, i.e. the taker when the ask quotes and the quoter otherwise.
// A self-trade or a zero quantity changes nothing, so it is skipped.
ASTRA_HD void apply_portfolio(int32_t *pf, int32_t C, int32_t price, int32_t qty, int32_t taker,
                              int32_t quoter, bool ask_quotes) {
  const int32_t buyer = ask_quotes ? taker : quoter, seller = ask_quotes ? quoter : taker;
  if (qty != 0 && (uint32_t)buyer < (uint32_t)C && (uint32_t)seller < (uint32_t)C &&
      buyer != seller) {
    const uint32_t notional = (uint32_t)price * (uint32_t)qty;
    add_i32(pf + 2 * buyer, qty);
    add_i32(pf + 2 * buyer + 1, (int32_t)(0u - notional));
    add_i32(pf + 2 * seller, (int32_t)(0u - (uint32_t)qty));
    add_i32(pf + 2 * seller + 1, (int32_t)notional);
  }
}

// Fill rows a lane has produced but not yet written. On the GPU the rows live
// in LDS as [field][row][lane] (a row write by 64 lanes touches 64 consecutive
// words: no bank conflicts); the host build keeps them in a local array. Rows
// go out R at a time (2 or 4, a template argument of the matching kernel) as
// aligned vector stores (rows k..k+R-1 of one market are contiguous in each
// field array), together with the portfolio updates they imply. Nothing beyond
// the call's last row is ever written: the reference leaves later entries of a
// FillBatch untouched.
template <int R>
struct FillSink {
  static_assert(R == 2 || R == 4, "two or four rows");
#if defined(__HIP_DEVICE_COMPILE__)
  int32_t *lds;  // this wavefront's [8][R][64] buffer
  int lane;
  __device__ int32_t &at(int f, int r) const { return lds[(f * R + r) * 64 + lane]; }
#else
  mutable int32_t buf[8][R];
  int32_t &at(int f, int r) const { return buf[f][r]; }
#endif
  int64_t base = 0;  // fill index of buffered row 0
  int32_t n = 0;     // rows buffered

  ASTRA_HD void flush(const FillOut &out, int32_t *pf, int32_t C) {
    if (n == 0) return;
    if (out.rows) {
      for (int r = 0; r < n; ++r) {
        int32_t v[8];
#pragma unroll
        for (int f = 0; f < 8; ++f) v[f] = at(f, r);
        write_row(out.rows, base + r, v);
      }
      for (int r = 0; r < n; ++r)
        apply_portfolio(pf, C, at(0, r), at(1, r), at(2, r), at(3, r), at(4, r) != 0);
      base += n;
      n = 0;
      return;
    }
    int32_t *dst32[7] = {out.prices, out.sizes, out.taker, out.quoter, out.quote_sizes, out.tid,
                         out.quote_tid};
    const int fidx[7] = {0, 1, 2, 3, 5, 6, 7};
#pragma unroll
    for (int j = 0; j < 7; ++j) {
      int32_t *d = dst32[j] + base;
      const int f = fidx[j];
      const uintptr_t a = reinterpret_cast<uintptr_t>(d);
      if (R == 4 && (a & 15) == 0) {  // rows k..k+3 of a 4-row-aligned run
        if (n == 4) {
          gst(reinterpret_cast<int4 *>(d), make_int4(at(f, 0), at(f, 1), at(f, 2), at(f, 3)));
        } else if (n == 3) {  // one 12-byte store instead of an 8- and a 4-byte one
          gst(reinterpret_cast<int3 *>(d), make_int3(at(f, 0), at(f, 1), at(f, 2)));
        } else {
          if (n & 2) gst(reinterpret_cast<int2 *>(d), make_int2(at(f, 0), at(f, 1)));
          if (n & 1) gst(d + (n - 1), at(f, n - 1));
        }
      } else if (R == 2 && n == 2 && (a & 7) == 0) {
        gst(reinterpret_cast<int2 *>(d), make_int2(at(f, 0), at(f, 1)));
      } else {
        for (int r = 0; r < n; ++r) gst(d + r, at(f, r));
      }
    }
    uint8_t *d8 = out.is_sell_quote + base;
    const uintptr_t a8 = reinterpret_cast<uintptr_t>(d8);
    if (R == 4 && (a8 & 3) == 0) {
      if (n == 4) {
        gst(reinterpret_cast<uint32_t *>(d8),
            (uint32_t)at(4, 0) | ((uint32_t)at(4, 1) << 8) | ((uint32_t)at(4, 2) << 16) |
                ((uint32_t)at(4, 3) << 24));
      } else {
        if (n & 2)
          gst(reinterpret_cast<uint16_t *>(d8),
              (uint16_t)((uint32_t)at(4, 0) | ((uint32_t)at(4, 1) << 8)));
        if (n & 1) gst(d8 + (n - 1), (uint8_t)at(4, n - 1));
      }
    } else if (R == 2 && n == 2 && (a8 & 1) == 0) {
      gst(reinterpret_cast<uint16_t *>(d8), (uint16_t)((uint32_t)at(4, 0) | ((uint32_t)at(4, 1) << 8)));
    } else {
      for (int r = 0; r < n; ++r) gst(d8 + r, (uint8_t)at(4, r));
    }
    for (int r = 0; r < n; ++r)
      apply_portfolio(pf, C, at(0, r), at(1, r), at(2, r), at(3, r), at(4, r) != 0);
    base += n;
    n = 0;
  }

  ASTRA_HD bool full() const { return false; }  // flushes itself

  ASTRA_HD void put(const FillOut &out, int32_t *pf, int32_t C, const int32_t (&row)[8]) {
#pragma unroll
    for (int f = 0; f < 8; ++f) at(f, n) = row[f];
    if (++n == R) flush(out, pf, C);
  }

};

// Rows of the one market being finished on a staged book (LDS on the GPU),
// kept short: {bid head slot | ask head slot << 16, quantity, the resting
// order's size before the fill, 0}, one 16-byte write per row on the lane
// that walks the book. The rest of a row (prices, customers, TIDs) is in the
// two heads' records, which a walk never changes (it changes sizes only), so
// the whole wavefront rebuilds the rows from the staged records when it writes
// them out (flush_rows). When the buffer is full the walk stops, the rows go
// out, and the walk resumes.
constexpr int32_t kStageRows = 128;

struct RowBuffer {
  uint4 *rows;
  int32_t cap;
  int32_t n;
  int64_t base;  // fill index of row 0
  ASTRA_HD bool full() const { return n == cap; }
  ASTRA_HD int32_t put_fill(const FillOut &, int32_t *, int32_t, const uint4 &b, const uint4 &a,
                            uint32_t bh, uint32_t ah, int32_t qty) {
    const bool bid_quote = (int32_t)b.z < (int32_t)a.z;  // as make_row
    rows[n] = make_uint4(bh | (ah << 16), (uint32_t)qty, bid_quote ? b.x : a.x, 0u);
    ++n;
    return (int32_t)((bid_quote ? b.w : a.w) & kNull16);
  }
};

// Rows [first, n) of a row buffer, `step` rows apart (64 lanes: row r by lane
// r % 64, so each field's stores are coalesced), rebuilt from the staged
// records `srec`, with their portfolio updates.
ASTRA_HD void flush_rows(const FillOut &out, const uint4 *rows, const uint4 *srec, int32_t n,
                         int64_t base, int32_t *pf, int32_t C, int32_t first, int32_t step) {
  for (int32_t r = first; r < n; r += step) {
    const uint4 e = rows[r];
    uint4 b = srec[e.x & kNull16], a = srec[e.x >> 16];
    b.x = a.x = e.z;  // make_row takes the resting order's size from its record
    int32_t v[8];
    make_row(b, a, (int32_t)e.y, v);
    write_fill(out, base + r, v);
    apply_portfolio(pf, C, v[0], v[1], v[2], v[3], v[4] != 0);
  }
}

// What stays fixed for a market during its matching loop.
struct MarketCtx {
  int64_t m;
  int32_t L, O, F, C;
  uint16_t *lv;  // the market's level words and order records in global memory
  uint4 *rec;
  int32_t *pf;
  int32_t ns;             // ring position after the inserts
  int32_t tid;            // the call's TID base (bid: tid, ask: tid + 1)
  bool bid_ok, ask_ok;
  bool keep_b, keep_a;    // a head the call left untouched whose size the cache holds
  GameQuote gq;           // the game's move (GAME only)
  bool abort;             // GAME: a failed check stops the whole move
};

// The matching loop's state: everything a lane needs to resume the loop later.
template <int W>
struct LoopState {
  uint64_t bm[W], am[W];
  int bb, ba;                  // best levels
  uint32_t bh, ah;             // their head slots
  uint4 brec, arec;            // records of bh / ah when have_b / have_a
  bool have_b, have_a;
  int pb, pa;                  // next levels whose words were read ahead
  uint32_t pbh, pah;           // their head slots
  bool ahead;                  // read-ahead issued for the current levels
  int32_t fc;                  // fills so far (-1 after an overflow)
  int32_t last_px;             // price of the last fill row written
  uint32_t emptied, forwarded; // diagnostic counts
  uint32_t npass;
  uint32_t zruns, zrows;       // zero-size walks on a staged book and their rows
};

// What one step of a multi-step launch hands its market's next step, in
// registers: the market's coalesced words as the step's epilogue left them
// (masks, ring position, best-level heads and sizes), so the next prologue
// skips its first round trip, and the next step's quotes, loaded ahead.
// (The masks are carried for up to 256 levels; wider ones would spill
// registers, so those markets reload their coalesced words every step.)
template <int W>
struct Carry {
  static constexpr bool kState = W <= 4;
  uint64_t bm[W], am[W];
  int32_t ns, tid, bsz, asz;
  uint32_t tob;
  int32_t q[5];
  bool state, quotes;
};

// Step k's quotes of market m into the carry (nothing past the last step).
template <int W>
ASTRA_HD void load_next_quotes(const QuoteIn &in, int64_t M, int32_t k, int32_t steps, int64_t m,
                               Carry<W> &cy) {
  cy.quotes = k < steps;
  if (!cy.quotes) return;
  const int64_t o = (int64_t)k * M + m;
  cy.q[0] = in.bid_px[o];
  cy.q[1] = in.bid_sz[o];
  cy.q[2] = in.ask_px[o];
  cy.q[3] = in.ask_sz[o];
  cy.q[4] = in.cust[o];
}

// The book as the loop sees it. GlobalBook: the market's arrays in global
// memory. StagedBook: a copy of the market's records and level words (in LDS
// on the GPU) that the loop reads; its writes (order sizes, level words) go to
// the copy and through to global memory, so global memory is current when the
// walk ends and nothing is copied back (a walk changes a few words of a book of
// 17 KB at the config-3 shape).
struct GlobalBook {
  static constexpr bool kStaged = false;
  uint16_t *lv;
  uint4 *rec;
  ASTRA_HD uint4 record(uint32_t s) const { return rec[s]; }
  ASTRA_HD int32_t size(uint32_t s) const { return reinterpret_cast<const int32_t *>(rec + s)[0]; }
  ASTRA_HD uint32_t word(int32_t p, int side) const { return level_word(lv, p, side); }
  ASTRA_HD uint32_t head(int32_t p, int side) const { return level_head(lv, p, side); }
  ASTRA_HD void set_size(uint32_t s, int32_t v) const {
    reinterpret_cast<int32_t *>(rec + s)[0] = v;
  }
  ASTRA_HD void set_word(int32_t p, int side, uint32_t w) const { store_level_word(lv, p, side, w); }
  ASTRA_HD void set_head(int32_t p, int side, uint32_t h) const { store_head(lv, p, side, h); }
};

struct StagedBook {
  static constexpr bool kStaged = true;
  static constexpr bool kLean = true;  // the loop's lean runs (cross_run, zero_levels)
  uint16_t *slv;  // the copy
  uint4 *srec;
  uint16_t *glv;  // the market's arrays in global memory
  uint4 *grec;
  ASTRA_HD uint4 record(uint32_t s) const { return srec[s]; }
  ASTRA_HD int32_t size(uint32_t s) const { return reinterpret_cast<const int32_t *>(srec + s)[0]; }
  ASTRA_HD uint32_t word(int32_t p, int side) const { return level_word(slv, p, side); }
  ASTRA_HD uint32_t head(int32_t p, int side) const { return level_head(slv, p, side); }
  ASTRA_HD void set_size(uint32_t s, int32_t v) const {
    reinterpret_cast<int32_t *>(srec + s)[0] = v;
    gst(reinterpret_cast<int32_t *>(grec + s), v);
  }
  ASTRA_HD void set_word(int32_t p, int side, uint32_t w) const {
    store_level_word(slv, p, side, w);
    gst(reinterpret_cast<uint32_t *>(glv + (size_t)p * 4 + 2 * side), w);
  }
  ASTRA_HD void set_head(int32_t p, int side, uint32_t h) const {
    store_head(slv, p, side, h);
    gst(glv + (size_t)p * 4 + 2 * side, (uint16_t)h);
  }
};

// Wave-uniform copies of the first active lane's values (readfirstlane; the
// identity on the host). A staged market's loop runs on one lane of its
// wavefront; on values the compiler knows to be uniform its branches compile to
// scalar branches instead of exec-mask bookkeeping, which halves the time a
// pass takes there.
ASTRA_HD int32_t uni(int32_t v) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_readfirstlane(v);
#else
  return v;
#endif
}
ASTRA_HD uint32_t uni(uint32_t v) { return (uint32_t)uni((int32_t)v); }
ASTRA_HD uint64_t uni(uint64_t v) {
  return (uint64_t)uni((uint32_t)v) | ((uint64_t)uni((uint32_t)(v >> 32)) << 32);
}
ASTRA_HD int64_t uni(int64_t v) { return (int64_t)uni((uint64_t)v); }
ASTRA_HD bool uni(bool v) { return uni((int32_t)(v ? 1 : 0)) != 0; }
ASTRA_HD uint4 uni(const uint4 &v) { return make_uint4(uni(v.x), uni(v.y), uni(v.z), uni(v.w)); }

// A staged book whose reads are wave-uniform (for the loop run by one lane).
struct UniformStagedBook : StagedBook {
  ASTRA_HD uint4 record(uint32_t s) const { return uni(srec[s]); }
  ASTRA_HD int32_t size(uint32_t s) const {
    return uni(reinterpret_cast<const int32_t *>(srec + s)[0]);
  }
  ASTRA_HD uint32_t word(int32_t p, int side) const { return uni(level_word(slv, p, side)); }
  ASTRA_HD uint32_t head(int32_t p, int side) const { return uni(level_head(slv, p, side)); }
};

// The same without the loop's lean runs (the game's move kernel: their code
// costs it more registers than they save it time).
struct UniformStagedBookPlain : UniformStagedBook {
  static constexpr bool kLean = false;
};
struct StagedBookPlain : StagedBook {
  static constexpr bool kLean = false;
};

template <int W>
ASTRA_HD LoopState<W> uniform_state(const LoopState<W> &a) {
  LoopState<W> u;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    u.bm[i] = uni(a.bm[i]);
    u.am[i] = uni(a.am[i]);
  }
  u.bb = uni(a.bb);
  u.ba = uni(a.ba);
  u.bh = uni(a.bh);
  u.ah = uni(a.ah);
  u.brec = uni(a.brec);
  u.arec = uni(a.arec);
  u.have_b = uni(a.have_b);
  u.have_a = uni(a.have_a);
  u.pb = uni(a.pb);
  u.pa = uni(a.pa);
  u.pbh = uni(a.pbh);
  u.pah = uni(a.pah);
  u.ahead = uni(a.ahead);
  u.fc = uni(a.fc);
  u.last_px = uni(a.last_px);
  u.emptied = uni(a.emptied);
  u.forwarded = uni(a.forwarded);
  u.npass = uni(a.npass);
  u.zruns = uni(a.zruns);
  u.zrows = uni(a.zrows);
  return u;
}

// The fields of MarketCtx the matching loop reads, made uniform.
ASTRA_HD MarketCtx uniform_ctx(const MarketCtx &a) {
  MarketCtx u = a;
  u.m = uni(a.m);
  u.L = uni(a.L);
  u.O = uni(a.O);
  u.F = uni(a.F);
  u.C = uni(a.C);
  u.ns = uni(a.ns);
  return u;
}

// ---- hand-off of a market's loop to the workgroup's helper wavefront ----
//
// With helpers (quote_match_kernel's HELP > 0) each workgroup holds HELP
// market wavefronts and one helper wavefront. A market lane whose walk is long
// (a run of zero-size orders ahead, or many passes) packs its loop state at
// the top of a pass into a slot of an LDS queue and leaves the market to the
// helper, which finishes it from an LDS copy of the book while the market
// wavefront goes on with its other lanes. Per market wavefront the queue has
// kHandSlots slots of kSlotWords words, each with a flag word (kSlotFree,
// kSlotReady, or kSlotClosed once the helper has gone); then one done word per
// market wavefront.
constexpr int kHandSlots = 4;
constexpr int kSlotWords = 48;
constexpr uint32_t kSlotFree = 0u, kSlotReady = 1u, kSlotClosed = 2u;

// Never hands off (every kernel without helpers, and the host build).
struct NoHand {
  static constexpr bool kOn = false;
};

// The loop state at the top of a pass and the call context of market c.m, as
// words: what the helper needs to resume the loop and end the call.
template <int W>
ASTRA_HD void pack_slot(uint32_t *p, const LoopState<W> &s, const MarketCtx &c) {
  static_assert(4 * W + 28 <= kSlotWords, "slot too small for the masks");
  int i = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    p[i++] = (uint32_t)s.bm[w];
    p[i++] = (uint32_t)(s.bm[w] >> 32);
    p[i++] = (uint32_t)s.am[w];
    p[i++] = (uint32_t)(s.am[w] >> 32);
  }
  p[i++] = (uint32_t)s.bb;
  p[i++] = (uint32_t)s.ba;
  p[i++] = s.bh;
  p[i++] = s.ah;
  p[i++] = s.brec.x;
  p[i++] = s.brec.y;
  p[i++] = s.brec.z;
  p[i++] = s.brec.w;
  p[i++] = s.arec.x;
  p[i++] = s.arec.y;
  p[i++] = s.arec.z;
  p[i++] = s.arec.w;
  p[i++] = (s.have_b ? 1u : 0u) | (s.have_a ? 2u : 0u) | (s.ahead ? 4u : 0u) |
           (c.bid_ok ? 8u : 0u) | (c.ask_ok ? 16u : 0u) | (c.keep_b ? 32u : 0u) |
           (c.keep_a ? 64u : 0u);
  p[i++] = (uint32_t)s.pb;
  p[i++] = (uint32_t)s.pa;
  p[i++] = s.pbh;
  p[i++] = s.pah;
  p[i++] = (uint32_t)s.fc;
  p[i++] = (uint32_t)s.last_px;
  p[i++] = s.emptied;
  p[i++] = s.forwarded;
  p[i++] = s.npass;
  p[i++] = s.zruns;
  p[i++] = s.zrows;
  p[i++] = (uint32_t)c.m;
  p[i++] = (uint32_t)((uint64_t)c.m >> 32);
  p[i++] = (uint32_t)c.ns;
  p[i++] = (uint32_t)c.tid;
}

// The inverse of pack_slot; the rest of the context follows from the book.
template <int W>
ASTRA_HD void unpack_slot(const uint32_t *p, const Book &b, LoopState<W> &s, MarketCtx &c) {
  int i = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    s.bm[w] = (uint64_t)p[i] | ((uint64_t)p[i + 1] << 32);
    s.am[w] = (uint64_t)p[i + 2] | ((uint64_t)p[i + 3] << 32);
    i += 4;
  }
  s.bb = (int)p[i++];
  s.ba = (int)p[i++];
  s.bh = p[i++];
  s.ah = p[i++];
  s.brec = make_uint4(p[i], p[i + 1], p[i + 2], p[i + 3]);
  i += 4;
  s.arec = make_uint4(p[i], p[i + 1], p[i + 2], p[i + 3]);
  i += 4;
  const uint32_t f = p[i++];
  s.have_b = (f & 1u) != 0;
  s.have_a = (f & 2u) != 0;
  s.ahead = (f & 4u) != 0;
  c.bid_ok = (f & 8u) != 0;
  c.ask_ok = (f & 16u) != 0;
  c.keep_b = (f & 32u) != 0;
  c.keep_a = (f & 64u) != 0;
  s.pb = (int)p[i++];
  s.pa = (int)p[i++];
  s.pbh = p[i++];
  s.pah = p[i++];
  s.fc = (int32_t)p[i++];
  s.last_px = (int32_t)p[i++];
  s.emptied = p[i++];
  s.forwarded = p[i++];
  s.npass = p[i++];
  s.zruns = p[i++];
  s.zrows = p[i++];
  c.m = (int64_t)((uint64_t)p[i] | ((uint64_t)p[i + 1] << 32));
  i += 2;
  c.ns = (int32_t)p[i++];
  c.tid = (int32_t)p[i++];
  c.L = b.L;
  c.O = b.O;
  c.F = b.F;
  c.C = b.C;
  c.lv = b.levels + c.m * (int64_t)b.L * 4;
  c.rec = b.records + c.m * (int64_t)b.O;
  c.pf = b.portfolios + c.m * (int64_t)b.C * 2;
  c.abort = false;
}

// A market wavefront's end of the queue.
struct Hand {
  static constexpr bool kOn = true;
  uint32_t *slots;     // this wavefront's kHandSlots slots
  uint32_t *flags;     // their flag words
  uint32_t *queue;     // the flag words of every slot of the workgroup, then the
                       // helper's busy word
  int32_t queued;      // flag words in `queue`
  int32_t max_queue;   // no hand-off while this many markets wait for the helper or
                       // are being finished by it
  int32_t threshold;   // passes after which any walk is handed off
  int32_t zero_lanes;  // a zero-size walk is handed off when at most this many lanes loop
  bool handed;         // this lane's market went to the helper
};

#if defined(__HIP_DEVICE_COMPILE__)
// The value, hidden from the optimiser (it cannot fold branches on it).
__device__ __forceinline__ bool opaque(bool v) {
  int32_t x = v ? 1 : 0;
  asm volatile("" : "+v"(x));
  return x != 0;
}

// Called at the top of a pass by the lanes still in their loop (records loaded,
// nothing of the pass done). Lanes that want to hand off take the free slots in
// lane order; a lane that gets one writes its buffered rows, packs its state and
// publishes the slot with a compare-and-swap from free to ready, which fails
// only when the helper has closed the slot meanwhile (it gave up waiting, below):
// the lane then keeps its market. Lanes left without a slot go on and ask again
// next pass.
template <int W, class Sink>
__device__ bool hand_off(Hand &h, bool want, const LoopState<W> &s, const MarketCtx &c, Sink &sink,
                         const FillOut &out) {
  const uint64_t req = __ballot(want);
  if (req == 0) return false;
  // markets already with the helper (waiting, or the one it is finishing): a
  // long queue would keep this one waiting longer than its walk takes in
  // global memory
  int32_t waiting = 0;
  for (int j = 0; j <= h.queued; ++j)
    waiting += (int32_t)__hip_atomic_load(h.queue + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  waiting = uni(waiting);
  uint32_t freem = 0;
#pragma unroll
  for (int j = 0; j < kHandSlots; ++j)
    freem |= (__hip_atomic_load(h.flags + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u
                  ? 1u
                  : 0u)
             << j;
  freem = uni(freem);
  if (!want || freem == 0 || waiting >= h.max_queue) return false;
  const int room = h.max_queue - waiting;
  const int k = (int)__popcll(req & ((1ull << __lane_id()) - 1ull));
  if (k >= __popc(freem) || k >= room) return false;
  uint32_t f = freem;
  for (int i = 0; i < k; ++i) f &= f - 1u;
  const int j = __ffs(f) - 1;
  // the helper read the slot before it freed it
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  sink.flush(out, c.pf, c.C);
  pack_slot<W>(h.slots + j * kSlotWords, s, c);
  // the book's writes, the rows and the slot before the flag
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  uint32_t expect = kSlotFree;
  if (!__hip_atomic_compare_exchange_strong(h.flags + j, &expect, kSlotReady, __ATOMIC_RELAXED,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))
    return false;  // closed: the helper has gone, the lane goes on with its market
  h.handed = true;
  return true;
}
#endif

// add_orders_kernel (market.cu:17-100) for market m and the set-up of the
// matching loop (:122-142): masks, the inserts, the heads of the best levels
// and their records.
//
// A lane waits on memory round trips, so the prologue takes two. The first
// reads the market's coalesced words: quotes, masks, ring position, and the
// head slots of the best levels as the last call left them (tob). That fixes
// the best levels after the inserts and whether the book crosses. The second
// reads the two insert levels' words and, for a market that crosses (or whose
// head sizes the call hands out), the two head records and the next level of
// each side, all at once, before the inserts write anything; the values are
// then patched for what the inserts wrote (a slot the ring reuses, a tail
// link), so the first loop pass starts with everything in registers.
template <int W, bool GAME, bool CARRY = false>
ASTRA_HD void quote_prologue(const Book &b, const QuoteIn &in, int64_t m, MarketCtx &c,
                             LoopState<W> &s, const Carry<W> *cy = nullptr) {
  const int64_t M = b.M;
  const int32_t L = b.L, O = b.O;
  c.m = m;
  c.L = L;
  c.O = O;
  c.F = b.F;
  c.C = b.C;
  c.lv = b.levels + m * (int64_t)L * 4;
  c.rec = b.records + m * (int64_t)O;
  c.pf = b.portfolios + m * (int64_t)b.C * 2;
  uint16_t *lv = c.lv;
  uint4 *rec = c.rec;

  // ---- round trip 1 ----
  int32_t bid_px, bid_sz, ask_px, ask_sz, cust;
  if (CARRY && cy->quotes) {
    bid_px = cy->q[0];
    bid_sz = cy->q[1];
    ask_px = cy->q[2];
    ask_sz = cy->q[3];
    cust = cy->q[4];
  } else if (GAME) {
    c.gq = game_quote(in.game, m);
    bid_px = c.gq.bid_px;
    bid_sz = c.gq.bid_sz;
    ask_px = c.gq.ask_px;
    ask_sz = c.gq.ask_sz;
    cust = in.game.player;
  } else {
    bid_px = in.bid_px[m];
    bid_sz = in.bid_sz[m];
    ask_px = in.ask_px[m];
    ask_sz = in.ask_sz[m];
    cust = in.cust[m];
  }
  // The head sizes of the best levels (for the BBO of a book that does not
  // cross) are only wanted where the call returns the BBO itself (the game
  // move, a multi-step launch); get_bbos reads them from the book otherwise.
  constexpr bool kSizes = GAME || CARRY;
  int32_t ns, bsz0 = 0, asz0 = 0;
  uint32_t tob;
  const bool carried = CARRY && Carry<W>::kState && cy->state;
  if (carried) {
#pragma unroll
    for (int i = 0; i < W; ++i) {
      s.bm[i] = cy->bm[i];
      s.am[i] = cy->am[i];
    }
    ns = cy->ns;
    c.tid = cy->tid;
    tob = cy->tob;
    bsz0 = cy->bsz;
    asz0 = cy->asz;
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) {
      s.bm[i] = b.masks[(int64_t)i * M + m];
      s.am[i] = b.masks[(int64_t)(W + i) * M + m];
    }
    ns = b.next_slot[m];
    c.tid = b.tids[m];
    tob = b.tob[m];
  }
  GameSnap snap;
  if (GAME) snap = game_snapshot(in.game, c.pf);
  c.abort = GAME && in.game.abort_on_error && *in.game.errors != 0;
  if (GAME && c.abort) return;  // nothing written yet
  if (GAME) game_before(in.game, snap, c.pf, m, c.gq.bad);

  const bool bid_ok = bid_sz > 0 && (uint32_t)bid_px < (uint32_t)L;
  const bool ask_ok = ask_sz > 0 && (uint32_t)ask_px < (uint32_t)L;
  const int bb0 = mask_highest<W>(s.bm);
  const int ba0 = mask_lowest<W>(s.am, L);
  // An insert above the best bid (below the best ask) lands on an empty level
  // and becomes that side's best level with the new order as head.
  const bool bid_top = bid_ok && bid_px > bb0;
  const bool ask_top = ask_ok && ask_px < ba0;
  const int bb = bid_top ? bid_px : bb0;
  const int ba = ask_top ? ask_px : ba0;
  const bool cross = bb >= 0 && ba < L && bb >= ba;
  const uint32_t hb0f = tob & kNull16, ha0f = tob >> 16;  // with their size flags
  const uint32_t hb0 = hb0f == kNull16 ? kNull16 : (hb0f & ~kSizeKnown);
  const uint32_t ha0 = ha0f == kNull16 ? kNull16 : (ha0f & ~kSizeKnown);

  // ---- round trip 2 ----
  // The insert levels' words: unconditional loads (level 0 stands in for a
  // rejected quote) so that nothing waits on them before the loads below are
  // issued; conditional ones each cost a round trip of their own.
  const uint32_t bword_ld = level_word(lv, bid_ok ? bid_px : 0, 0);
  const uint32_t aword_ld = level_word(lv, ask_ok ? ask_px : 0, 1);
  const uint32_t bword = bid_ok ? bword_ld : 0u;
  const uint32_t aword = ask_ok ? aword_ld : 0u;
  uint4 hrb = make_uint4((uint32_t)bsz0, 0, 0, 0), hra = make_uint4((uint32_t)asz0, 0, 0, 0);
  // Head records read here: a crossing book's, all where the call hands out the
  // BBO, and a head whose size the cache does not hold (so that this call's
  // epilogue caches it and get_bbos, every step until the head changes, reads
  // no record for it).
  const bool head_recs = cross || (kSizes && !carried);
  const bool load_b = !bid_top && hb0 < (uint32_t)O && (head_recs || !(hb0f & kSizeKnown));
  const bool load_a = !ask_top && ha0 < (uint32_t)O && (head_recs || !(ha0f & kSizeKnown));
  if (load_b) hrb = rec[hb0];
  if (load_a) hra = rec[ha0];
  int pb = -1, pa = L;
  uint32_t pbh = kNull16, pah = kNull16;
  if (cross) {
    uint64_t t[W];
#pragma unroll
    for (int i = 0; i < W; ++i) t[i] = s.bm[i];
    if (bid_ok) mask_set<W>(t, bid_px);
    mask_clear<W>(t, bb);
    pb = mask_highest<W>(t);
    if (pb >= 0) pbh = level_head(lv, pb, 0);
#pragma unroll
    for (int i = 0; i < W; ++i) t[i] = s.am[i];
    if (ask_ok) mask_set<W>(t, ask_px);
    mask_clear<W>(t, ba);
    pa = mask_lowest<W>(t, L);
    if (pa < L) pah = level_head(lv, pa, 1);
  }

  // ---- add: bid first, then ask (market.cu:44-70, 73-99) ----
  uint32_t bslot = 0xFFFFFFFFu, aslot = 0xFFFFFFFFu;
  uint32_t btail = 0xFFFFFFFFu, atail = 0xFFFFFFFFu;  // old tails the inserts linked from
  uint4 krb = make_uint4(0, 0, 0, 0), kra = make_uint4(0, 0, 0, 0);
  if (bid_ok) {
    bslot = (uint32_t)ns;
    ns = (ns + 1 == O) ? 0 : ns + 1;
    krb = make_uint4((uint32_t)bid_sz, (uint32_t)cust, (uint32_t)c.tid,
                     (uint32_t)bid_px | (kNull16 << 16));
    rec[bslot] = krb;
    const uint32_t old_tail = bword >> 16;
    if (old_tail == kNull16) {
      store_level_word(lv, bid_px, 0, bslot | (bslot << 16));
      mask_set<W>(s.bm, bid_px);
    } else {
      lv[(size_t)bid_px * 4 + 1] = (uint16_t)bslot;
      if (old_tail < (uint32_t)O) {
        reinterpret_cast<uint16_t *>(rec + old_tail)[7] = (uint16_t)bslot;
        btail = old_tail;
      }
    }
  }
  if (ask_ok) {
    aslot = (uint32_t)ns;
    ns = (ns + 1 == O) ? 0 : ns + 1;
    kra = make_uint4((uint32_t)ask_sz, (uint32_t)cust, (uint32_t)((uint32_t)c.tid + 1u),
                     (uint32_t)ask_px | (kNull16 << 16));
    rec[aslot] = kra;
    const uint32_t old_tail = aword >> 16;
    if (old_tail == kNull16) {
      store_level_word(lv, ask_px, 1, aslot | (aslot << 16));
      mask_set<W>(s.am, ask_px);
    } else {
      lv[(size_t)ask_px * 4 + 3] = (uint16_t)aslot;
      if (old_tail < (uint32_t)O) {
        reinterpret_cast<uint16_t *>(rec + old_tail)[7] = (uint16_t)aslot;
        atail = old_tail;
      }
    }
  }
  // A record read before the inserts, as the inserts left it: the bid record
  // overwrites its slot, the bid links its old tail to it, then the same for
  // the ask (a slot can be both, e.g. O == 1).
  auto patched = [&](uint32_t slot, uint4 r) {
    if (slot == bslot) r = krb;
    if (slot == btail) r = with_next(r, bslot);
    if (slot == aslot) r = kra;
    if (slot == atail) r = with_next(r, aslot);
    return r;
  };
  c.ns = ns;
  c.bid_ok = bid_ok;
  c.ask_ok = ask_ok;

  // ---- the matching loop's entry state ----
  // For a market that does not cross only the head sizes are used, where the
  // call hands out the BBO; they come from the head records read above (or
  // the carry) unless an insert rewrote the slot.
  s.bb = bb;
  s.ba = ba;
  s.bh = s.ah = kNull16;
  s.brec = s.arec = make_uint4(0, 0, 0, 0);
  if (bb >= 0) {
    s.bh = bid_top ? bslot : hb0;
    s.brec = patched(s.bh, hrb);
  }
  if (ba < L) {
    s.ah = ask_top ? aslot : ha0;
    s.arec = patched(s.ah, hra);
  }
  // The head records in registers: read above, carried, or written by this
  // call's inserts. A head the call does not touch and whose record it did not
  // read keeps the size cached by an earlier call.
  const bool sizes_in = kSizes && carried;
  s.have_b = bb >= 0 && (sizes_in || bid_top || load_b || s.bh == bslot || s.bh == aslot);
  s.have_a = ba < L && (sizes_in || ask_top || load_a || s.ah == bslot || s.ah == aslot);
  c.keep_b = !cross && !s.have_b && bb >= 0 && !bid_top && hb0f != kNull16 && (hb0f & kSizeKnown) &&
             hb0 != 0x7FFFu;
  c.keep_a = !cross && !s.have_a && ba < L && !ask_top && ha0f != kNull16 && (ha0f & kSizeKnown) &&
             ha0 != 0x7FFFu;
  // the next levels read ahead, as the inserts left their heads
  if (bid_ok && pb == bid_px && (bword >> 16) == kNull16) pbh = bslot;
  if (ask_ok && pa == ask_px && (aword >> 16) == kNull16) pah = aslot;
  s.pb = pb;
  s.pa = pa;
  s.pbh = pbh;
  s.pah = pah;
  s.ahead = cross;
  s.fc = 0;
  s.last_px = 0;
  s.emptied = s.forwarded = s.npass = 0;
  s.zruns = s.zrows = 0;
}

// Passes in which one side's head has size 0 and the other side's a positive
// size: the fill is 0, nothing but that head changes, and it moves to the next
// order of its level (:237-256). Runs such passes back to back while the next
// order exists, differs from the current one and from the other head; writes
// the level's head once at the end. Called at the top of a pass with both
// records loaded; returns false when the budget or the sink stopped it (state
// intact at the top of a pass).
template <int SIDE, bool STATS, int W, class BookMem, class Sink>
ASTRA_HD bool zero_walk(LoopState<W> &s, const MarketCtx &c, const BookMem &bk, Sink &sink,
                        const FillOut &out, int32_t budget, int32_t &passes) {
  uint4 &w = SIDE == 0 ? s.brec : s.arec;
  uint32_t &h = SIDE == 0 ? s.bh : s.ah;
  const uint32_t start = h;
  bool ok = true;
  for (;;) {
    const uint32_t nh = rec_next(w);
    if (nh >= (uint32_t)c.O || nh == h || s.fc >= c.F) break;  // NULL (or out of range) ends it
    s.last_px = sink.put_fill(out, c.pf, c.C, s.brec, s.arec, s.bh, s.ah, 0);
    ++s.fc;
    if (STATS) ++s.zrows;
    h = nh;
    w = bk.record(nh);
    if (passes++ >= budget || sink.full()) {
      ok = false;
      break;
    }
    if ((int32_t)w.x != 0 || s.bh == s.ah) break;
  }
  if (h != start) {
    bk.set_head(SIDE == 0 ? s.bb : s.ba, SIDE, h);
    if (STATS) ++s.zruns;
  }
  return ok;
}

// On a staged book, passes whose one head has positive size and whose other
// head is an order of size 0 that is the last of its level (a consumed order
// still linked after ring-slot reuse): each fills 0 against it and empties its
// level (market.cu:196-273 with q = 0; the pop to the next level, :241-256 /
// :258-273). Runs such passes back to back while the side's next level holds
// such an order too and still crosses. Called at the top of a pass with both
// records loaded (the side's head of that kind, the other head of positive
// size, distinct heads, fills left); returns false when the budget or the sink
// stopped it (state intact at the top of a pass), else true with the state at
// the top of a pass.
template <int SIDE, bool STATS, int W, class BookMem, class Sink>
ASTRA_HD bool zero_levels(LoopState<W> &s, const MarketCtx &c, const BookMem &bk, Sink &sink,
                          const FillOut &out, int32_t budget, int32_t &passes) {
  uint4 &w = SIDE == 0 ? s.brec : s.arec;
  uint32_t &h = SIDE == 0 ? s.bh : s.ah;
  int &p = SIDE == 0 ? s.bb : s.ba;
  bool &have = SIDE == 0 ? s.have_b : s.have_a;
  uint64_t(&m)[W] = SIDE == 0 ? s.bm : s.am;
  const uint32_t other = SIDE == 0 ? s.ah : s.bh;
  const int32_t L = c.L;
  for (;;) {
    s.last_px = sink.put_fill(out, c.pf, c.C, s.brec, s.arec, s.bh, s.ah, 0);
    ++s.fc;
    if (STATS) {
      ++s.npass;
      ++s.emptied;
    }
    bk.set_word(p, SIDE, 0xFFFFFFFFu);
    mask_clear<W>(m, p);
    p = SIDE == 0 ? mask_highest<W>(m) : mask_lowest<W>(m, L);
    const bool live = SIDE == 0 ? p >= 0 : p < L;
    const uint32_t nh = bk.head(live ? p : 0, SIDE);
    h = live ? nh : kNull16;
    have = false;
    // the top of the next pass
    if (!live || s.bb < s.ba || h >= (uint32_t)c.O) return true;
    w = bk.record(h);
    have = true;
    if (h == other || (int32_t)w.x != 0 || rec_next(w) != kNull16 || s.fc >= c.F) return true;
    if (passes++ >= budget || sink.full()) return false;
  }
}

// On a staged book: passes of the crossing loop below run back to back while
// both heads are distinct orders of positive size (market.cu:196-273 for that
// case: the fill is the smaller size, both sizes drop by it, and a side whose
// size is then 0 pops to the next order of its level or, at the end of the
// level, to the next level). Size-0 heads are left to zero_walk and
// zero_levels, repeating and aliased states to the loop below. A pass of the
// loop below on a staged book costs ~1,600 cycles (one wavefront, one lane:
// instruction issue, taken branches and LDS round trips one after another);
// this run keeps its state in registers, reads both head records together
// once per pass, and writes a surviving order's size and a level's new head
// once, when the run ends or the level empties. Called at the top of a pass
// with both records loaded and the book crossing; returns whether it made a
// pass, and leaves every write in the book and the state at the top of a pass
// (the loop's next pass reads both records again).
template <int W, bool STATS, class BookMem, class Sink>
ASTRA_HD bool cross_run(LoopState<W> &s, const MarketCtx &c, const BookMem &bk, Sink &sink,
                        const FillOut &out, int32_t budget, int32_t &passes) {
  const int32_t L = c.L;
  const uint32_t O = (uint32_t)c.O;
  bool any = false;
  bool size_b = false, size_a = false;  // the head's size in the book is stale
  bool head_b = false, head_a = false;  // the level's head word is stale
  int32_t bsz = (int32_t)s.brec.x, asz = (int32_t)s.arec.x;
  for (;;) {
    if (s.bh == s.ah || bsz <= 0 || asz <= 0 || s.fc >= c.F) break;
    const uint32_t nb = rec_next(s.brec), na = rec_next(s.arec);
    if (any) {
      if (passes >= budget || sink.full()) break;
      ++passes;
    }
    any = true;
    if (STATS) ++s.npass;
    const int32_t qty = bsz < asz ? bsz : asz;
    s.last_px = sink.put_fill(out, c.pf, c.C, s.brec, s.arec, s.bh, s.ah, qty);
    ++s.fc;
    bsz -= qty;  // both >= 0: no wrap
    asz -= qty;
    const bool pop_b = bsz == 0, pop_a = asz == 0;
    size_b = !pop_b;  // (qty > 0: the size changed)
    size_a = !pop_a;
    s.brec.x = (uint32_t)bsz;
    s.arec.x = (uint32_t)asz;
    if (pop_b) {
      bk.set_size(s.bh, 0);
      if (nb == kNull16) {
        bk.set_word(s.bb, 0, 0xFFFFFFFFu);
        head_b = false;
        mask_clear<W>(s.bm, s.bb);
        if (STATS) ++s.emptied;
        s.bb = mask_highest<W>(s.bm);
        const uint32_t h = bk.head(s.bb >= 0 ? s.bb : 0, 0);
        s.bh = s.bb >= 0 ? h : kNull16;
      } else if (nb != s.bh) {
        s.bh = nb;
        head_b = true;
      }
      s.have_b = false;
    }
    if (pop_a) {
      bk.set_size(s.ah, 0);
      if (na == kNull16) {
        bk.set_word(s.ba, 1, 0xFFFFFFFFu);
        head_a = false;
        mask_clear<W>(s.am, s.ba);
        if (STATS) ++s.emptied;
        s.ba = mask_lowest<W>(s.am, L);
        const uint32_t h = bk.head(s.ba < L ? s.ba : 0, 1);
        s.ah = s.ba < L ? h : kNull16;
      } else if (na != s.ah) {
        s.ah = na;
        head_a = true;
      }
      s.have_a = false;
    }
    // the top of the next pass
    if (s.bb < 0 || s.ba >= L || s.bb < s.ba || s.bh >= O || s.ah >= O) break;
    // both records at once; a head that did not pop keeps its size (the book's
    // copy may be stale) and its other fields (which nothing changes)
    const uint4 rb = bk.record(s.bh), ra = bk.record(s.ah);
    s.brec = rb;
    s.arec = ra;
    bsz = pop_b ? (int32_t)rb.x : bsz;
    asz = pop_a ? (int32_t)ra.x : asz;
    s.brec.x = (uint32_t)bsz;
    s.arec.x = (uint32_t)asz;
    s.have_b = s.have_a = true;
  }
  if (size_b) bk.set_size(s.bh, (int32_t)s.brec.x);
  if (size_a) bk.set_size(s.ah, (int32_t)s.arec.x);
  if (head_b) bk.set_head(s.bb, 0, s.bh);
  if (head_a) bk.set_head(s.ba, 1, s.ah);
  return any;
}

// match_orders_kernel's crossing loop (market.cu:145-274). Runs at most
// `budget` passes and stops early when the sink is full, or (EARLY, in global
// memory) before a zero-size walk of a lane left nearly alone
// (kEarlyStageLanes); returns false (state intact, nothing of the next pass
// done) when it stopped before the end.
//
// Two loop states repeat forever (both arise from ring-slot reuse): a size-0
// head that links to itself (each pass emits the same zero-size fill and
// changes nothing) and one slot heading both sides with size s != 0 (fills of
// s and -s alternate). The reference loops until F fills and then writes -1;
// here the owed rows are handed to the caller in `bulk`, the final state is set
// directly, and the count is -1, which is the same result.
//
// With a Hand (helpers), a lane whose walk is long hands its market off at the
// top of a pass instead (returns false; hand->handed set).
template <int W, bool STATS, bool EARLY, class BookMem, class Sink, class HandT = NoHand>
ASTRA_HD bool match_loop(LoopState<W> &s, const MarketCtx &c, const BookMem &bk, Sink &sink,
                         const FillOut &out, Bulk &bulk, int32_t budget, HandT *hand = nullptr) {
  const int32_t L = c.L, O = c.O, F = c.F;
  int32_t passes = 0;
  while (s.bb >= 0 && s.ba < L && s.bb >= s.ba) {
    if (s.bh >= (uint32_t)O || s.ah >= (uint32_t)O) break;  // NULL head (:155)
    if (passes++ >= budget || sink.full()) return false;
    // Records of heads that changed (the entry heads come from the prologue);
    // every size change is written through, so memory is current.
    if constexpr (BookMem::kStaged) {
      // On the staged book a read costs instructions, not memory traffic: both
      // head records are read every pass, issued before one wait, and an
      // emptied level's successor is looked up when it empties (below), so the
      // read-ahead bookkeeping of the global-memory loop drops out.
      s.brec = bk.record(s.bh);
      s.arec = bk.record(s.ah);
      s.have_b = s.have_a = true;
    } else {
      if (!s.have_b) {
        s.brec = bk.record(s.bh);
        s.have_b = true;
      }
      if (!s.have_a) {
        s.arec = bk.record(s.ah);
        s.have_a = true;
      }
      if (!s.ahead) {  // read the next level of each side ahead
        uint64_t t[W];
#pragma unroll
        for (int i = 0; i < W; ++i) t[i] = s.bm[i];
        mask_clear<W>(t, s.bb);
        s.pb = mask_highest<W>(t);
#pragma unroll
        for (int i = 0; i < W; ++i) t[i] = s.am[i];
        mask_clear<W>(t, s.ba);
        s.pa = mask_lowest<W>(t, L);
        // both heads in one round trip: unconditional loads (level 0 stands in
        // for a side with no next level), nothing waits on them in this block
        s.pbh = bk.head(s.pb >= 0 ? s.pb : 0, 0);
        s.pah = bk.head(s.pa < L ? s.pa : 0, 1);
        s.ahead = true;
      }
      // A lane that is one of at most kEarlyStageLanes still looping in its
      // wavefront and is about to walk a run of zero-size orders stops here
      // when staging is enabled: each further pass would cost the wavefront a
      // memory round trip (3-4 us under load), while the staged book walks
      // such a run at instruction speed (0.2 us a row). Lanes that still have
      // company go on: the wavefront waits for them anyway. (At most 1, 2, 4,
      // 8 or any lane: 2 is fastest at 100,000 and 10,000 markets.)
      if constexpr (HandT::kOn) {
#if defined(__HIP_DEVICE_COMPILE__)
        const bool zstart = s.bh != s.ah && (((int32_t)s.brec.x == 0 && (int32_t)s.arec.x > 0) ||
                                             ((int32_t)s.arec.x == 0 && (int32_t)s.brec.x > 0));
        const bool want =
            passes > hand->threshold || (zstart && lanes_here() <= hand->zero_lanes);
        // (opaque: otherwise the compiler moves the slot's writes and its flag
        // onto the loop's exit path, which runs only when every lane of the
        // wavefront has left the loop, and the helper would see nothing before)
        if (opaque(hand_off<W>(*hand, want, s, c, sink, out))) return false;
#endif
      } else if constexpr (EARLY) {
        const int32_t looping = lanes_here();
        if (budget != 0x7FFFFFFF && looping <= kEarlyStageLanes && s.bh != s.ah &&
            (((int32_t)s.brec.x == 0 && (int32_t)s.arec.x > 0) ||
             ((int32_t)s.arec.x == 0 && (int32_t)s.brec.x > 0)))
          return false;
      }
    }
    // On the staged book a pass costs instructions, not memory round trips,
    // so the short zero-size walk pays there (in global memory it does not).
    if constexpr (BookMem::kStaged) {
      if (s.bh != s.ah) {
        if ((int32_t)s.brec.x == 0 && (int32_t)s.arec.x > 0) {
          if (!zero_walk<0, STATS>(s, c, bk, sink, out, budget, passes)) return false;
        } else if ((int32_t)s.arec.x == 0 && (int32_t)s.brec.x > 0) {
          if (!zero_walk<1, STATS>(s, c, bk, sink, out, budget, passes)) return false;
        }
      }
      if constexpr (BookMem::kLean) {
        if (s.bh != s.ah && s.fc < F) {
          if ((int32_t)s.brec.x == 0 && rec_next(s.brec) == kNull16 && (int32_t)s.arec.x > 0) {
            if (!zero_levels<0, STATS>(s, c, bk, sink, out, budget, passes)) return false;
            continue;
          }
          if ((int32_t)s.arec.x == 0 && rec_next(s.arec) == kNull16 && (int32_t)s.brec.x > 0) {
            if (!zero_levels<1, STATS>(s, c, bk, sink, out, budget, passes)) return false;
            continue;
          }
        }
        if (cross_run<W, STATS>(s, c, bk, sink, out, budget, passes)) continue;
      }
    }
    if (STATS) ++s.npass;
    const int32_t bsz = (int32_t)s.brec.x, asz = (int32_t)s.arec.x;
    const int32_t qty = bsz < asz ? bsz : asz;
    if (s.fc >= F) {  // overflow sentinel (:187-195)
      s.fc = -1;
      break;
    }
    // In global memory the row is made here (kept in registers for the sink and
    // the repeat cases); on a staged book the row buffer keeps a short form.
    int32_t row[8];
    if constexpr (!BookMem::kStaged) make_row(s.brec, s.arec, qty, row);
    if (s.bh == s.ah && bsz != 0) {
      // One slot heads both sides with size s != 0: q = s, the slot becomes -s,
      // neither side pops, and the next pass is the same with -s. The fills
      // alternate s, -s until F; the trade is a self-trade (no portfolio
      // change); the slot ends at s or -s by the parity of the fill count.
      bulk.base = c.m * (int64_t)F + s.fc;
      bulk.count = F - s.fc;
      bulk.alt = 1;
      if constexpr (BookMem::kStaged) {
        make_row(s.brec, s.arec, qty, bulk.v);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) bulk.v[i] = row[i];
      }
      const int32_t fin = ((F - s.fc) & 1) ? (int32_t)(0u - (uint32_t)bsz) : bsz;
      bk.set_size(s.bh, fin);
      s.brec.x = s.arec.x = (uint32_t)fin;
      s.fc = -1;
      if (STATS) ++s.forwarded;
      break;
    }
    // the row and its portfolio update (:198-232)
    if constexpr (BookMem::kStaged) {
      s.last_px = sink.put_fill(out, c.pf, c.C, s.brec, s.arec, s.bh, s.ah, qty);
    } else {
      sink.put(out, c.pf, c.C, row);
      s.last_px = row[0];
    }
    ++s.fc;
    // (:237-238) both decrements land on one slot when bid and ask alias
    if (s.bh == s.ah) {
      const int32_t sz = wsub(wsub(bsz, qty), qty);
      s.brec.x = s.arec.x = (uint32_t)sz;
      if (qty != 0) bk.set_size(s.bh, sz);
    } else {
      s.brec.x = (uint32_t)wsub(bsz, qty);
      s.arec.x = (uint32_t)wsub(asz, qty);
      if (qty != 0) {
        bk.set_size(s.bh, (int32_t)s.brec.x);
        bk.set_size(s.ah, (int32_t)s.arec.x);
      }
    }
    const uint32_t bh_was = s.bh, ah_was = s.ah;
    const int bb_was = s.bb, ba_was = s.ba;
    if (s.brec.x == 0u) {  // pop the bid head (:241-256)
      const uint32_t nh = rec_next(s.brec);
      if (nh == kNull16) {
        bk.set_word(s.bb, 0, 0xFFFFFFFFu);
        mask_clear<W>(s.bm, s.bb);
        if (STATS) ++s.emptied;
        if constexpr (BookMem::kStaged) {  // the highest remaining level and its head
          s.bb = mask_highest<W>(s.bm);
          s.bh = s.bb >= 0 ? bk.head(s.bb, 0) : kNull16;
        } else {
          // the next level is the one read ahead at the top of this pass (pb
          // is the highest level below bb in the same mask, and only this pop
          // has changed the mask since)
          s.bb = s.pb;
          s.bh = s.bb >= 0 ? (s.pbh & kNull16) : kNull16;
        }
        s.have_b = false;
        s.ahead = false;
      } else if (nh != s.bh) {
        bk.set_head(s.bb, 0, nh);
        s.bh = nh;
        s.have_b = false;
      }
    }
    if (s.arec.x == 0u) {  // pop the ask head (:258-273)
      const uint32_t nh = rec_next(s.arec);
      if (nh == kNull16) {
        bk.set_word(s.ba, 1, 0xFFFFFFFFu);
        mask_clear<W>(s.am, s.ba);
        if (STATS) ++s.emptied;
        if constexpr (BookMem::kStaged) {  // the lowest remaining level and its head
          s.ba = mask_lowest<W>(s.am, L);
          s.ah = s.ba < L ? bk.head(s.ba, 1) : kNull16;
        } else {
          s.ba = s.pa;
          s.ah = s.ba < L ? (s.pah & kNull16) : kNull16;
        }
        s.have_a = false;
        s.ahead = false;
      } else if (nh != s.ah) {
        bk.set_head(s.ba, 1, nh);
        s.ah = nh;
        s.have_a = false;
      }
    }
    if (qty == 0 && s.bh == bh_was && s.ah == ah_was && s.bb == bb_was && s.ba == ba_was) {
      // Nothing changed (a size-0 head linked to itself): every further pass
      // writes this same row until F. Portfolios and sizes are untouched.
      bulk.base = c.m * (int64_t)F + s.fc;
      bulk.count = F - s.fc;
      bulk.alt = 0;
      if constexpr (BookMem::kStaged) {
        // (the heads and their records are the pass's: so is the row)
        make_row(s.brec, s.arec, 0, bulk.v);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) bulk.v[i] = row[i];
      }
      s.fc = -1;
      if (STATS) ++s.forwarded;
      break;
    }
  }
  return true;
}

// The end of a market's call: remaining fill rows, fill count, masks, ring
// position, and the best levels of the book as left (prices into the
// workspace's BBO cache, head slots into tob: what get_bbo_kernel,
// market.cu:280-320, would find). STATS also adds the call's work counts.
template <int W, bool STATS, bool GAME, bool MULTI, class BookMem, class Sink>
ASTRA_HD void quote_epilogue(const Book &b, const FillOut &out, const MarketCtx &c,
                             const LoopState<W> &s, Sink &sink, const BookMem &bk,
                             const GameMove &game, const StepOut &so,
                             Carry<W> *cy = nullptr, bool last = true) {
  const int64_t M = b.M, m = c.m;
  const int32_t L = c.L, O = c.O;
  // Loads first, then plain stores and the fill rows with their portfolio
  // atomics, then the stores that need the loaded values: the wait for a load
  // also waits for every memory operation issued before it.
  // The head sizes (GetBBOs' sizes) only where this call hands out the BBO:
  // loading them ends a chain with one more round trip.
  constexpr bool kSizes = GAME || MULTI;
  int32_t obs = 0, oas = 0;
  if (kSizes && s.bb >= 0 && s.bh < (uint32_t)O) obs = s.have_b ? (int32_t)s.brec.x : bk.size(s.bh);
  if (kSizes && s.ba < L && s.ah < (uint32_t)O) oas = s.have_a ? (int32_t)s.arec.x : bk.size(s.ah);
  gst(out.counts + m, s.fc);
  // (a multi-step launch keeps these in registers and stores them after its
  // last step only)
  const bool store = !MULTI || last || !Carry<W>::kState;
  if (store) {
#pragma unroll
    for (int i = 0; i < W; ++i) {
      b.masks[(int64_t)i * M + m] = s.bm[i];
      b.masks[(int64_t)(W + i) * M + m] = s.am[i];
    }
    b.next_slot[m] = c.ns;
    b.tids[m] = (int32_t)((uint32_t)c.tid + 2u);  // market.cu:531
  }
  sink.flush(out, c.pf, c.C);  // overlaps the loads above
  const bool bv = s.bb >= 0 && s.bh < (uint32_t)O, av = s.ba < L && s.ah < (uint32_t)O;
  const int32_t obp = bv ? s.bb : ASTRA_NULL_INDEX;
  const int32_t oap = av ? s.ba : ASTRA_NULL_INDEX;
  // Head sizes the call knows (the record is in registers, or the call hands
  // out the BBO and loaded it) go to the size cache; a head the call left
  // untouched keeps the size an earlier call cached. get_bbos reads the book
  // only for the others.
  // (slot 0x7FFF, possible at O = 32768, is never flagged: flagged it would read
  // as NULL)
  // (on a staged book a head's record is an LDS read away: every head's size is
  // cached there)
  bool hb = s.have_b, ha = s.have_a;
  int32_t bsz_c = (int32_t)s.brec.x, asz_c = (int32_t)s.arec.x;
  if constexpr (BookMem::kStaged && !kSizes) {
    if (!hb && bv) {
      bsz_c = bk.size(s.bh);
      hb = true;
    }
    if (!ha && av) {
      asz_c = bk.size(s.ah);
      ha = true;
    }
  }
  const bool wb = bv && (kSizes || hb) && s.bh != 0x7FFFu;
  const bool wa = av && (kSizes || ha) && s.ah != 0x7FFFu;
  const uint32_t tob = (bv ? (s.bh | ((wb || c.keep_b) ? kSizeKnown : 0u)) : kNull16) |
                       ((av ? (s.ah | ((wa || c.keep_a) ? kSizeKnown : 0u)) : kNull16) << 16);
  if (store) {
    b.bbo[m] = obp;
    b.bbo[M + m] = oap;
    b.tob[m] = tob;
    if (wb) b.hsz[m] = kSizes ? obs : bsz_c;
    if (wa) b.hsz[M + m] = kSizes ? oas : asz_c;
  }
  if (MULTI && Carry<W>::kState && cy) {
#pragma unroll
    for (int i = 0; i < W; ++i) {
      cy->bm[i] = s.bm[i];
      cy->am[i] = s.am[i];
    }
    cy->ns = c.ns;
    cy->tid = (int32_t)((uint32_t)c.tid + 2u);
    cy->tob = tob;
    cy->bsz = obs;
    cy->asz = oas;
    cy->state = true;
  }
  if (GAME) {
    const int32_t bbo[4] = {obp, obs, oap, oas};
    game_after(game, c.gq, c.pf, M, m, bbo, s.fc, s.last_px);
  }
  if (MULTI) {
    if (so.counts) so.counts[m] = s.fc;
    if (so.bbo[0]) {
      so.bbo[0][m] = obp;
      so.bbo[1][m] = obs;
      so.bbo[2][m] = oap;
      so.bbo[3][m] = oas;
    }
  }

  if (STATS) {  // uniform addresses: the compiler aggregates these per wave
    add_u64(b.stats + 0, (unsigned long long)(c.bid_ok + c.ask_ok));
    add_u64(b.stats + 1, (unsigned long long)(s.fc < 0 ? c.F : s.fc));
    add_u64(b.stats + 2, (unsigned long long)s.emptied);
    add_u64(b.stats + 3, (unsigned long long)(s.fc < 0));
    add_u64(b.stats + 4, (unsigned long long)s.forwarded);
    add_u64(b.stats + 5, (unsigned long long)s.npass);
    add_u64(b.stats + 6, (unsigned long long)(BookMem::kStaged ? 1 : 0));
    add_u64(b.stats + 7, (unsigned long long)(s.npass > 0 ? 1 : 0));
    add_u64(b.stats + 8, (unsigned long long)s.zruns);
    add_u64(b.stats + 9, (unsigned long long)s.zrows);
    add_u64(b.stats + 10, (unsigned long long)((bv && !wb && !c.keep_b) + (av && !wa && !c.keep_a)));
  }
}

// GetBBOs (market.cu:573-597) reads the cache the last call left: the best
// level and the size of its head order per side, (NULL, 0) for an empty side.
// Sizes come from the head-size cache where the tob word flags them, else from
// the head order's record in the book.
ASTRA_HD void bbo_copy_market(const Book &b, int32_t *bid_px, int32_t *bid_sz, int32_t *ask_px,
                              int32_t *ask_sz, int64_t m) {
  const int64_t M = b.M;
  const int32_t bp = b.bbo[m], ap = b.bbo[M + m];
  const uint32_t t = b.tob[m], bf = t & kNull16, af = t >> 16;
  const int32_t cb = b.hsz[m], ca = b.hsz[M + m];
  const uint32_t bh = bf & ~kSizeKnown, ah = af & ~kSizeKnown;
  const bool bv = bp != ASTRA_NULL_INDEX && bf != kNull16 && bh < (uint32_t)b.O;
  const bool av = ap != ASTRA_NULL_INDEX && af != kNull16 && ah < (uint32_t)b.O;
  const uint4 *rec = b.records + m * (int64_t)b.O;
  int32_t bs = cb, as = ca;
  if (bv && !(bf & kSizeKnown)) bs = reinterpret_cast<const int32_t *>(rec + bh)[0];
  if (av && !(af & kSizeKnown)) as = reinterpret_cast<const int32_t *>(rec + ah)[0];
  bid_px[m] = bp;
  ask_px[m] = ap;
  bid_sz[m] = bv ? bs : 0;
  ask_sz[m] = av ? as : 0;
}

// update_last_prices_kernel (market.cu:767-786). A count above F (only possible
// for caller-made fill_counts) leaves the last price unchanged.
ASTRA_HD void last_price_market(int32_t *last, const int32_t *counts, const int32_t *prices,
                                int32_t F, int32_t stride, int64_t m) {
  const int32_t c = counts[m];
  if (c > 0 && c <= F) last[m] = prices[(m * (int64_t)F + (c - 1)) * stride];
}

// ClearQuotes (market.cu:735-749) for thread t = (market, level): the level's
// 8-byte word to all-NULL; the level-0 thread also zeroes the masks and the slot
// counter and empties the market's BBO cache. The reference also writes NULL
// into order_next; here a slot's next is
// overwritten whenever the slot is reused, and after the clear no list can
// reach a slot that was not reused, so it is left alone (no observable
// difference).
template <int W>
ASTRA_HD void clear_quotes_thread(const Book &b, const uint8_t *reset, int64_t t) {
  const int64_t per = b.L > 0 ? b.L : 1;
  const int64_t m = t / per;
  const int64_t p = t - m * per;
  if (m >= b.M || !reset[m]) return;
  const int64_t M = b.M;
  if (p < b.L) reinterpret_cast<uint64_t *>(b.levels)[m * (int64_t)b.L + p] = ~0ull;
  if (p == 0) {
#pragma unroll
    for (int i = 0; i < 2 * W; ++i) b.masks[(int64_t)i * M + m] = 0ull;
    b.next_slot[m] = 0;
    b.bbo[m] = ASTRA_NULL_INDEX;
    b.bbo[M + m] = ASTRA_NULL_INDEX;
    b.tob[m] = 0xFFFFFFFFu;
  }
}

// ---- __global__ wrappers ----

// A pointer moved into vector registers, opaque to the compiler so that it stays
// there (the identity on the host). The matching kernel keeps every kernel
// argument in scalar registers and has more of them live in its loop than
// there are: the fill-batch pointers (used by the row flushes) go to VGPRs,
// which the kernel has to spare, instead of being spilled and reloaded around
// each branch of the loop (-1.5% per step at 100,000 markets, -4.5% at 10,000;
// not in the game move's kernel, which has no VGPRs to spare).
template <class T>
__device__ __forceinline__ T *in_vgpr(T *p) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint64_t v = reinterpret_cast<uint64_t>(p);
  asm volatile("" : "+v"(v));
  return reinterpret_cast<T *>(v);
#else
  return p;
#endif
}

// ---- the TID counter in device memory ----
//
// The reference keeps one TID counter on the host and passes the base as a
// kernel argument (market.cu:520,531), which a launch captured in a HIP graph
// would replay frozen. Here every market keeps the counter in a word of its own
// (Book::tids): a call reads it with the market's other coalesced words and
// writes it back advanced in its epilogue. Every call steps every market, so
// all the words hold the same value, the reference's counter; no lane waits on
// another and a captured launch replays with advancing TIDs.

// The counter's advance of a call on zero markets (no matching launch).
__global__ void tid_advance_kernel(int32_t *ctl, int32_t by) {
  if (threadIdx.x == 0)
    __hip_atomic_store(ctl + kCtlTid, (int32_t)((uint32_t)ctl[kCtlTid] + (uint32_t)by),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Writes the rows owed by fast-forwarded markets of this wavefront: each such
// lane's rows are written by all 64 lanes together, coalesced.
__device__ __forceinline__ void write_bulk_wave(const FillOut &out, const Bulk &bk) {
  uint64_t pending = __ballot(bk.count > 0);
  const int lane = (int)__lane_id();
  while (pending) {
    const int src = __ffsll((unsigned long long)pending) - 1;
    pending &= pending - 1;
    const int32_t base_lo = __shfl((int32_t)(uint32_t)bk.base, src);
    const int32_t base_hi = __shfl((int32_t)(bk.base >> 32), src);
    const int64_t base = (int64_t)(((uint64_t)(uint32_t)base_hi << 32) | (uint32_t)base_lo);
    const int32_t count = __shfl(bk.count, src);
    const int32_t alt = __shfl(bk.alt, src);
    int32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __shfl(bk.v[i], src);
    for (int32_t k = lane; k < count; k += 64) {
      int32_t r[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = v[i];
      if (alt && (k & 1)) {
        r[1] = (int32_t)(0u - (uint32_t)r[1]);
        r[5] = (int32_t)(0u - (uint32_t)r[5]);
      }
      write_fill(out, base + k, r);
    }
  }
}

// All 64 lanes of a wavefront reach write_bulk_wave (no early return).
// LDS per wavefront: the fill-row buffer and (when staging is enabled for the
// shape) the staged book of one market, side by side where the whole grid
// still fits on the CUs that way, else sharing one area (the book overwrites
// the buffer after the lanes have written their rows out).
ASTRA_HD constexpr size_t sink_bytes(int32_t rows) { return (size_t)8 * rows * 64 * sizeof(int32_t); }
typedef __attribute__((address_space(1))) void gvoid_t;  // global memory
typedef __attribute__((address_space(3))) void lvoid_t;  // LDS

// Staged book of one market: records, level words (padded to 16 bytes), then
// its row buffer.
ASTRA_HD size_t stage_bytes(int32_t L, int32_t O) {
  return (size_t)O * 16 + ((size_t)L * 8 + 15) / 16 * 16 + (size_t)kStageRows * sizeof(uint4);
}

ASTRA_HD int64_t shfl_i64(int64_t v, int src) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int32_t lo = __shfl((int32_t)(uint32_t)v, src);
  const int32_t hi = __shfl((int32_t)((uint64_t)v >> 32), src);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
#else
  (void)src;
  return v;
#endif
}

// Finishes lane src's market from a copy of its book in LDS (`stage`: the
// records, the level words padded to 16 bytes, then the row buffer). The whole
// wavefront copies the book in with coalesced loads, the owning lane resumes
// its loop reading the copy (on wave-uniform copies of its state), and all 64
// lanes write the rows out, coalesced, each time the row buffer fills and at
// the end; then the owning lane writes the call's epilogue. All 64 lanes call
// this together.
template <int W, bool STATS, bool GAME, bool MULTI, class Sink>
__device__ void finish_staged(const Book &b, const FillOut &out, int32_t *stage, int lane, int src,
                              int64_t m, MarketCtx &c, LoopState<W> &st, Sink &sink, Bulk &bulk,
                              const GameMove &game, const StepOut &sok, Carry<W> *cy, bool last) {
  const int64_t ms = shfl_i64(m, src);
  uint4 *srec = reinterpret_cast<uint4 *>(stage);
  uint64_t *slv = reinterpret_cast<uint64_t *>(srec + b.O);
  uint4 *rows = reinterpret_cast<uint4 *>(slv + ((b.L + 1) & ~1));  // 16-byte aligned
  uint4 *grec = b.records + ms * (int64_t)b.O;
  uint64_t *glv = reinterpret_cast<uint64_t *>(b.levels) + ms * (int64_t)b.L;
  int32_t *pfm = b.portfolios + ms * (int64_t)b.C * 2;
  __builtin_amdgcn_wave_barrier();
#if defined(__HIP_DEVICE_COMPILE__)
  // LDS DMA (global_load_lds): each lane's 16 (or 4) bytes go straight to LDS
  // at the wave-uniform base + lane * size, no registers involved, all loads
  // in flight together. The records are loaded non-temporal (cache policy 2, nt):
  // a staged book's 16 KB is read once, and kept out of the way of the other
  // wavefronts' record reads (2% off config 3's step).
  for (int32_t j = 0; j < b.O; j += 64)
    if (j + lane < b.O)
      __builtin_amdgcn_global_load_lds((gvoid_t *)(grec + j + lane), (lvoid_t *)(srec + j), 16, 0,
                                       2);
  const uint32_t *glv32 = reinterpret_cast<const uint32_t *>(glv);
  uint32_t *slv32 = reinterpret_cast<uint32_t *>(slv);
  for (int32_t j = 0; j < 2 * b.L; j += 64)
    if (j + lane < 2 * b.L)
      __builtin_amdgcn_global_load_lds((gvoid_t *)(glv32 + j + lane), (lvoid_t *)(slv32 + j), 4, 0,
                                       0);
  __builtin_amdgcn_s_waitcnt(0);
#endif
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  std::conditional_t<GAME, UniformStagedBookPlain, UniformStagedBook> sb;
  sb.slv = reinterpret_cast<uint16_t *>(slv);
  sb.srec = srec;
  sb.glv = reinterpret_cast<uint16_t *>(glv);
  sb.grec = grec;
  RowBuffer rb{rows, kStageRows, 0, 0};
  if (lane == src) rb.base = sink.base;
  // The owning lane runs until its market is done or its row buffer is full
  // (on uniform copies of its state); then all 64 lanes write the rows out.
  bool done = false;
  while (!done) {
    int32_t fin = 0;
    if (lane == src) {
      LoopState<W> us = uniform_state(st);
      const MarketCtx uc = uniform_ctx(c);
      RowBuffer urb{rows, kStageRows, uni(rb.n), uni(rb.base)};
      fin = match_loop<W, STATS, false>(us, uc, sb, urb, out, bulk, 0x7FFFFFFF) ? 1 : 0;
      st = us;
      rb.n = urb.n;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int32_t n = __shfl(rb.n, src);
    const int64_t base = shfl_i64(rb.base, src);
    done = uni(__shfl(fin, src) != 0);
    flush_rows(out, rows, srec, n, base, pfm, b.C, lane, 64);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == src) {
      rb.base += n;
      rb.n = 0;
    }
  }
  if (lane == src) {
    sink.base = rb.base;
    quote_epilogue<W, STATS, GAME, MULTI>(b, out, c, st, sink, sb, game, sok, cy, last);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Idle polls before a helper wavefront gives up waiting (the default of the
// launch's `helper_polls`): far beyond any market wavefront's lifetime (each
// poll sleeps about 0.1 us), it only bounds the kernel if a market wavefront
// never signalled its end.
constexpr int32_t kHelperMaxPolls = 1 << 22;

// The helper wavefront of a workgroup with H market wavefronts: takes ready
// slots of the queue in LDS (lowest first), frees each slot once its state is
// read, finishes the market (finish_staged, lane 0 walking) and writes its
// repeating rows; returns when every market wavefront has signalled its end and
// no slot is ready.
//
// After `max_polls` idle polls in a row it gives up instead: it closes every
// free slot (a compare-and-swap from free to closed, so a market lane's
// publication either comes first and is finished here, or fails and the lane
// keeps its market), finishes the markets already published, counts the
// give-up in the workspace's control words and returns. Every market is then
// finished, by the helper or in global memory by its own lane.
template <int W, int H>
__device__ void helper_wave(const Book &b, const FillOut &out, int32_t *stage, uint32_t *slots,
                            uint32_t *flags, const uint32_t *done, int lane, int32_t max_polls) {
  uint32_t *busy = flags + H * kHandSlots;  // 1 while a market is being finished
  FillSink<4> sink;  // never buffers a row: the epilogue's flush finds it empty
#if defined(__HIP_DEVICE_COMPILE__)
  sink.lds = stage;
  sink.lane = lane;
#endif
  // finishes the market in slot j; the slot becomes `after` once it is read
  auto take = [&](int j, uint32_t after) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    LoopState<W> st;
    MarketCtx c;
    unpack_slot<W>(slots + j * kSlotWords, b, st, c);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) {
      __hip_atomic_store(busy, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_store(flags + j, after, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    sink.n = 0;
    sink.base = c.m * (int64_t)b.F + st.fc;
    Bulk bulk;
    bulk.count = 0;
    finish_staged<W, false, false, false>(b, out, stage, lane, 0, c.m, c, st, sink, bulk,
                                          GameMove{}, StepOut{}, (Carry<W> *)nullptr, true);
    if (lane != 0) bulk.count = 0;
    write_bulk_wave(out, bulk);
    if (lane == 0) __hip_atomic_store(busy, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  int32_t polls = 0;
  for (;;) {
    uint32_t ready = 0;
#pragma unroll
    for (int j = 0; j < H * kHandSlots; ++j)
      ready |= (__hip_atomic_load(flags + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) ==
                        kSlotReady
                    ? 1u
                    : 0u)
               << j;
    ready = uni(ready);
    if (ready) {
      take(__ffs(ready) - 1, kSlotFree);
      polls = 0;
      continue;
    }
    uint32_t ended = 0;
#pragma unroll
    for (int i = 0; i < H; ++i)
      ended += __hip_atomic_load(done + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (uni(ended) == (uint32_t)H) {
      // every slot published before a done word is ready by now
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      uint32_t left = 0;
#pragma unroll
      for (int j = 0; j < H * kHandSlots; ++j)
        left |= __hip_atomic_load(flags + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (uni(left) == 0u) return;
      continue;
    }
    if (uni(++polls) > max_polls) break;
    __builtin_amdgcn_s_sleep(2);
  }
  // Give up: lane 0 closes every free slot (one compare-and-swap each); a slot
  // that was ready instead is finished here and closed once read. After this
  // one pass no slot can become ready, so the wavefront finishes the ones found
  // ready in a loop over a wave-uniform mask (every lane takes part in
  // finish_staged's cooperative copy; a loop whose condition the compiler
  // takes for divergent has run the second finish on lane 0 alone).
  uint32_t ready = 0;
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < H * kHandSlots; ++j) {
      uint32_t expect = kSlotFree;
      if (!__hip_atomic_compare_exchange_strong(flags + j, &expect, kSlotClosed, __ATOMIC_RELAXED,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) &&
          expect == kSlotReady)
        ready |= 1u << j;
    }
  }
  for (uint32_t pending = uni((uint32_t)__shfl((int32_t)ready, 0)); pending; pending &= pending - 1u)
    take(__ffs(pending) - 1, kSlotClosed);
  if (lane == 0)
    __hip_atomic_fetch_add(b.ctl + kCtlHelperExits, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Fused add + match + BBO, one lane per market, in two passes.
//   1. Every lane runs its market's loop for at most `budget` passes (or
//      fewer: see kEarlyStageLanes).
//   2. Markets still crossing after that (long walks through stale or
//      consumed orders) are finished one at a time: the whole wavefront copies
//      the market's order records and level words into LDS with coalesced
//      loads, and the owning lane resumes its loop reading from LDS.
// MULTI runs `steps` consecutive calls in one launch: markets are independent,
// so each wavefront goes on to its markets' next step as soon as it is done
// with this one, with no grid-wide wait between steps.
// FR: fill rows a lane buffers before writing them (fill_rows_per_flush). With
// FR = 2 (small grids) a staged book has LDS of its own beside the row buffer,
// and the finished lanes' epilogues come after the staged walks: a staged
// book's copy-in ends with a wait for every memory operation the wavefront has
// in flight (loads and stores share one counter), so stores issued before it
// delay it. With FR = 4 the book reuses the row buffer's LDS (the whole grid of
// a large launch fits on the CUs only that way), so the finished lanes write
// their epilogues, rows included, before it.
// HELP > 0 (large grids, FR = 4, single-step calls): each workgroup is HELP
// market wavefronts and one helper wavefront, and step 2 runs on the helper
// instead, concurrently with the market wavefronts' loops: a lane whose walk is
// long (`budget` passes, or a run of zero-size orders ahead while at most
// `hand_lanes` lanes of its wavefront still loop) hands its market over
// through an LDS queue (hand_off, helper_wave) and its wavefront goes on. LDS
// per workgroup: the HELP row buffers, the helper's staged book, the queue.
// All 64 lanes of a wavefront reach the ballots (no early return but the
// helper wavefront's, which returns as a whole).
template <int W, bool STATS, bool GAME, bool MULTI, bool ROWS, int FR, int HELP = 0>
__global__ __launch_bounds__(256) void quote_match_kernel(Book b, QuoteIn in, FillOut out,
                                                          StepOut so, int32_t steps,
                                                          int32_t budget, int32_t wave_words,
                                                          int32_t per_wave, int32_t hand_lanes,
                                                          int32_t hand_queue, int32_t helper_polls) {
  constexpr bool kApart = FR == 2;  // the staged book beside the row buffer
  static_assert(HELP == 0 || (!STATS && !GAME && !MULTI && FR == 4 && W <= 4),
                "helpers serve plain single-step calls of large grids");
  extern __shared__ int32_t lds_words[];
  // The FillBatch layout is a template argument: the other layout's pointers
  // become constant nulls, so their code and registers drop out.
  if (ROWS) {
    out.prices = out.sizes = out.taker = out.quoter = nullptr;
    out.quote_sizes = out.tid = out.quote_tid = nullptr;
    out.is_sell_quote = nullptr;
    if (!GAME) out.rows = in_vgpr(out.rows);
  } else {
    out.rows = nullptr;
    if (!GAME) {
      out.prices = in_vgpr(out.prices);
      out.sizes = in_vgpr(out.sizes);
      out.taker = in_vgpr(out.taker);
      out.quoter = in_vgpr(out.quoter);
      out.is_sell_quote = in_vgpr(out.is_sell_quote);
      out.quote_sizes = in_vgpr(out.quote_sizes);
      out.tid = in_vgpr(out.tid);
      out.quote_tid = in_vgpr(out.quote_tid);
    }
  }
  if (!GAME) out.counts = in_vgpr(out.counts);
  // Lanes [0, per_wave) of each wavefront own one market each; the rest idle
  // (and help with the wavefront's cooperative copies).
  const int lane = (int)(threadIdx.x % 64);
  const int wv = (int)uni((int32_t)(threadIdx.x / 64));  // wavefront within the workgroup
  Hand hand{nullptr, nullptr, nullptr, 0, hand_queue, budget, hand_lanes, false};
  if constexpr (HELP > 0) {
    int32_t *stage = lds_words + HELP * wave_words;
    uint32_t *slots = reinterpret_cast<uint32_t *>(stage + stage_bytes(b.L, b.O) / 4);
    uint32_t *flags = slots + HELP * kHandSlots * kSlotWords;
    uint32_t *done = flags + HELP * kHandSlots + 1;  // after the helper's busy word
    if (threadIdx.x < HELP * (kHandSlots + 1) + 1) flags[threadIdx.x] = 0u;
    __syncthreads();
    if (wv == HELP) {
      helper_wave<W, HELP>(b, out, stage, slots, flags, done, lane, helper_polls);
      return;
    }
    hand.slots = slots + wv * kHandSlots * kSlotWords;
    hand.flags = flags + wv * kHandSlots;
    hand.queue = flags;
    hand.queued = HELP * kHandSlots;
  }
  const int64_t wave = HELP > 0 ? (int64_t)blockIdx.x * HELP + wv
                                : ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / 64;
  const int64_t m = lane < per_wave ? wave * per_wave + lane : b.M;
  int32_t *wave_lds = lds_words + wv * wave_words;
  FillSink<FR> sink;
#if defined(__HIP_DEVICE_COMPILE__)
  sink.lds = wave_lds;
  sink.lane = lane;
#endif
  Carry<W> cy;
  cy.state = cy.quotes = false;
  for (int32_t k = 0; k < (MULTI ? steps : 1); ++k) {
    QuoteIn ink = in;
    StepOut sok = so;
    if (MULTI) step_views(in, so, b.M, steps, k, ink, sok);
    const bool last = k + 1 == (MULTI ? steps : 1);
    Bulk bulk;
    bulk.count = 0;
    MarketCtx c;
    LoopState<W> st;
    bool suspended = false, finished = false;
    if (m < b.M) quote_prologue<W, GAME, MULTI>(b, ink, m, c, st, &cy);
    if (MULTI && m < b.M) load_next_quotes(in, b.M, k + 1, steps, m, cy);
    if (m < b.M && !(GAME && c.abort)) {
      sink.base = m * (int64_t)b.F;
      const GlobalBook gb{c.lv, c.rec};
      if constexpr (HELP > 0) {
        // the loop ends here or hands the market to the helper
        if (match_loop<W, STATS, false>(st, c, gb, sink, out, bulk, 0x7FFFFFFF, &hand))
          quote_epilogue<W, STATS, GAME, MULTI>(b, out, c, st, sink, gb, ink.game, sok, &cy, last);
      } else if (match_loop<W, STATS, !GAME>(st, c, gb, sink, out, bulk, budget)) {
        if constexpr (kApart) {
          finished = true;
          // The records of heads the loop moved to without reading them, loaded
          // now so that the epilogue after the staged walks caches their sizes
          // (get_bbos then reads no record for this market): the loads complete
          // while the wavefront stages its walks, off its critical path.
          if (!GAME && !MULTI) {
            const uint32_t O = (uint32_t)c.O;
            if (!st.have_b && st.bb >= 0 && st.bh < O && st.bh != 0x7FFFu) {
              st.brec = gb.record(st.bh);
              st.have_b = true;
            }
            if (!st.have_a && st.ba < c.L && st.ah < O && st.ah != 0x7FFFu) {
              st.arec = gb.record(st.ah);
              st.have_a = true;
            }
          }
        } else
          quote_epilogue<W, STATS, GAME, MULTI>(b, out, c, st, sink, gb, ink.game, sok, &cy, last);
      } else {
        sink.flush(out, c.pf, c.C);  // the staged walk's rows follow these
        suspended = true;
      }
    }
    uint64_t todo = HELP > 0 ? 0ull : __ballot(suspended);
    while (todo) {
      const int src = __ffsll((unsigned long long)todo) - 1;
      todo &= todo - 1;
      finish_staged<W, STATS, GAME, MULTI>(b, out, wave_lds + (kApart ? sink_bytes(FR) / 4 : 0), lane,
                                           src, m, c, st, sink, bulk, ink.game, sok, &cy, last);
    }
    if constexpr (kApart) {
      if (finished)
        quote_epilogue<W, STATS, GAME, MULTI>(b, out, c, st, sink, GlobalBook{c.lv, c.rec},
                                              ink.game, sok, &cy, last);
    }
    write_bulk_wave(out, bulk);
    if constexpr (HELP > 0) {  // this wavefront has handed off all it will
      uint32_t *done = hand.flags - wv * kHandSlots + HELP * kHandSlots + 1;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) __hip_atomic_store(done + wv, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (MULTI) {  // this step's rows and book writes come before the next step's
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

__global__ __launch_bounds__(256) void bbo_kernel(Book b, int32_t *bid_px, int32_t *bid_sz,
                                                  int32_t *ask_px, int32_t *ask_sz) {
  const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m < b.M) bbo_copy_market(b, bid_px, bid_sz, ask_px, ask_sz, m);
}

__global__ __launch_bounds__(256) void last_price_kernel(int32_t *last, const int32_t *counts,
                                                         const int32_t *prices, int32_t M,
                                                         int32_t F, int32_t stride) {
  const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m < M) last_price_market(last, counts, prices, F, stride, m);
}

template <int W>
__global__ __launch_bounds__(256) void clear_quotes_kernel(Book b, const uint8_t *reset,
                                                           int64_t n) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) clear_quotes_thread<W>(b, reset, t);
}

// Grid-stride fill of n 32-bit words; 16-byte stores when dst is 16-byte aligned.
__global__ __launch_bounds__(kFillThreads) void fill_u32_kernel(uint32_t *dst, int64_t n,
                                                                uint32_t v, int vec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n4 = vec ? n / 4 : 0;
  uint4 *d4 = reinterpret_cast<uint4 *>(dst);
  const uint4 v4 = make_uint4(v, v, v, v);
  for (int64_t i = t; i < n4; i += stride) d4[i] = v4;
  for (int64_t i = n4 * 4 + t; i < n; i += stride) dst[i] = v;
}

// ---- launchers (kernel on the device build, host loop on the emulation build) ----

inline unsigned grid_for(int64_t n, int block) { return (unsigned)((n + block - 1) / block); }

// Markets per wavefront of the matching kernel: the handle's setting
// (ASTRA_MARKET_PER_WAVE at creation, 1-64) if any, else 64, or 32 for a game
// move over at most 65,536 envs (2,048 half-full wavefronts, what 256 CUs hold
// at 8 each): at 10,000 envs the 157 full wavefronts leave most SIMDs idle,
// and half-full ones end sooner (each waits for the slowest of fewer markets),
// 6% faster per move on MI355X; a grid that fills the GPU (config 3) is 6%
// slower at 32.
int32_t markets_per_wave(const astra_market *h, bool game) {
  if (h->per_wave) return h->per_wave;
  return (game && h->M <= 32 * 2048) ? 32 : 64;
}

// Fill rows a lane buffers before writing them: 2 where each CU holds at most
// two of the grid's wavefronts, 4 above. Under light load the rows that remain
// buffered at the end of a lane's chain are stores its wavefront waits out at
// the end; flushing every 2 rows leaves fewer (with the staged book's own LDS
// and the deferred epilogues: -5% after the ring wraps at 10,000 markets of the
// config-3 shape, -3% at config 4, -7.5% for the config-5 game move). Under
// full load every flush inside the loop costs the whole wavefront issue slots
// (+10% before the ring wraps at 100,000 markets), so 4 there.
int32_t fill_rows_per_flush(const astra_market *h, int64_t waves_per_cu) {
  if (h->fill_rows) return h->fill_rows;
  return waves_per_cu <= 2 ? 2 : 4;
}

template <int W, bool GAME, bool MULTI>
int launch_quote_match(const astra_market *h, const QuoteIn &in, const FillOut &fo,
                       const StepOut &so, int32_t steps, hipStream_t s) {
  const Book b = book_of(h);
  // Staging needs each wavefront's copy of a book (its records, level words
  // and row buffers) in LDS, within what a workgroup may use on the device
  // (160 KB on gfx950).
  const bool staged = h->stage_budget > 0 &&
                      (size_t)(h->block / 64) * align_up(stage_bytes(h->L, h->O), 16) <=
                          (size_t)h->lds_limit;
  const int32_t budget = staged ? h->stage_budget : 0x7FFFFFFF;
  const size_t stage_b = staged ? align_up(stage_bytes(h->L, h->O), 16) : (size_t)0;
  int32_t per_wave = markets_per_wave(h, GAME);
  // A single-step grid of at most one full wavefront per CU leaves most SIMDs
  // idle: half-full wavefronts end sooner (each waits for the slowest of fewer
  // markets), where the doubled grid still fits on the CUs at once with the
  // small grids' LDS per wavefront (config 2, 10,000 markets: +4%; at config 4
  // the doubled grid would not fit and run in two rounds).
  if (!h->per_wave && !GAME && !MULTI && (int64_t)b.M <= (int64_t)64 * h->cus) {
    const size_t wb = sink_bytes(2) + stage_b;
    const int64_t resident = (int64_t)h->cus * (int64_t)((size_t)h->lds_per_cu / wb);
    if (2 * (((int64_t)b.M + 63) / 64) <= resident) per_wave = 32;
  }
  // A multi-step launch of such a grid halves it down to 16 markets per
  // wavefront while the grid still fits on the CUs at once (its wavefronts
  // buffer 4 rows, in the LDS their staged books reuse): each wavefront's
  // steps wait for its slowest market, so fewer markets end each step sooner
  // (config 2, 10,000 markets, 20 steps: 5.3e8 at 64, 5.5e8 at 32, 5.7e8 at
  // 16; config 4 stays at 64, where 32 would not fit and is 30% slower).
  if (!h->per_wave && !GAME && MULTI && (int64_t)b.M <= (int64_t)64 * h->cus) {
    const size_t wb = std::max(sink_bytes(4), stage_b);
    const int64_t resident = (int64_t)h->cus * (int64_t)((size_t)h->lds_per_cu / wb);
    while (per_wave > 16 && ((int64_t)b.M + per_wave / 2 - 1) / (per_wave / 2) <= resident)
      per_wave /= 2;
  }
  const int64_t waves = ((int64_t)b.M + per_wave - 1) / per_wave;
  const int64_t waves_per_cu = (waves + h->cus - 1) / h->cus;
  // (a multi-step launch buffers 4: its wavefronts go on to the next step; and 2
  // only where the staged book fits beside the row buffer for every wavefront
  // the grid puts on a CU)
  const size_t apart_block = (size_t)(h->block / 64) * (sink_bytes(2) + stage_b);
  const bool fits_apart = apart_block <= (size_t)h->lds_limit &&
                          (int64_t)((size_t)h->lds_per_cu / apart_block) * (h->block / 64) >= waves_per_cu;
  const int32_t rows_cap = (MULTI || !fits_apart) ? 4 : fill_rows_per_flush(h, waves_per_cu);
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  const QuoteIn &inb = in;
  std::vector<uint4> srec(staged ? (size_t)h->O : 0);
  std::vector<uint16_t> slv(staged ? (size_t)h->L * 4 : 0);
  std::vector<uint4> rows((size_t)kStageRows);
  std::vector<Carry<W>> carry(MULTI ? (size_t)b.M : 0);
  for (auto &cy : carry) cy.state = cy.quotes = false;
  // one market's call, with a fill-row buffer of the launch's depth
  auto market = [&](auto sink, const QuoteIn &ink, const StepOut &sok, int32_t k, bool last,
                    int64_t m) {
    Bulk bulk;
    bulk.count = 0;
    MarketCtx c;
    LoopState<W> st;
    Carry<W> *cy = MULTI ? &carry[(size_t)m] : nullptr;
    quote_prologue<W, GAME, MULTI>(b, ink, m, c, st, cy);
    if (MULTI) load_next_quotes(inb, b.M, k + 1, steps, m, *cy);
    if (GAME && c.abort) return;
    sink.base = m * (int64_t)b.F;
    const GlobalBook gb{c.lv, c.rec};
    const bool done = b.stats ? match_loop<W, true, !GAME>(st, c, gb, sink, fo, bulk, budget)
                              : match_loop<W, false, !GAME>(st, c, gb, sink, fo, bulk, budget);
    if (done) {
      if (b.stats) quote_epilogue<W, true, GAME, MULTI>(b, fo, c, st, sink, gb, ink.game, sok, cy, last);
      else quote_epilogue<W, false, GAME, MULTI>(b, fo, c, st, sink, gb, ink.game, sok, cy, last);
    } else {  // the second pass, as on the GPU
      sink.flush(fo, c.pf, c.C);
      if constexpr (!GAME && W <= 4) {  // through a queue slot, as a hand-off to a helper would
        uint32_t slot[kSlotWords];
        pack_slot<W>(slot, st, c);
        unpack_slot<W>(slot, b, st, c);
      }
      std::memcpy(srec.data(), c.rec, (size_t)h->O * 16);
      std::memcpy(slv.data(), c.lv, (size_t)h->L * 8);
      std::conditional_t<GAME, StagedBookPlain, StagedBook> sb;
      sb.slv = slv.data();
      sb.srec = srec.data();
      sb.glv = c.lv;
      sb.grec = c.rec;
      RowBuffer rb{rows.data(), kStageRows, 0, sink.base};
      bool fin = false;
      while (!fin) {
        fin = b.stats ? match_loop<W, true, false>(st, c, sb, rb, fo, bulk, 0x7FFFFFFF)
                      : match_loop<W, false, false>(st, c, sb, rb, fo, bulk, 0x7FFFFFFF);
        flush_rows(fo, rows.data(), srec.data(), rb.n, rb.base, c.pf, c.C, 0, 1);
        rb.base += rb.n;
        rb.n = 0;
      }
      sink.base = rb.base;
      if (b.stats) quote_epilogue<W, true, GAME, MULTI>(b, fo, c, st, sink, sb, ink.game, sok, cy, last);
      else quote_epilogue<W, false, GAME, MULTI>(b, fo, c, st, sink, sb, ink.game, sok, cy, last);
    }
    if (bulk.count > 0) write_bulk_host(fo, bulk);
  };
  for (int32_t k = 0; k < (MULTI ? steps : 1); ++k) {
    QuoteIn ink = inb;
    StepOut sok = so;
    if (MULTI) step_views(inb, so, b.M, steps, k, ink, sok);
    const bool last = k + 1 == (MULTI ? steps : 1);
    for (int64_t m = 0; m < b.M; ++m) {
      if (rows_cap == 2) market(FillSink<2>{}, ink, sok, k, last, m);
      else market(FillSink<4>{}, ink, sok, k, last, m);
    }
  }
#else
  const size_t sink_b = sink_bytes(rows_cap);
  // Helpers (single-step calls of plain large grids whose books stage): HELP
  // market wavefronts and a helper per workgroup, if every workgroup the grid
  // puts on a CU still fits in its LDS.
  if constexpr (W <= 4 && !GAME && !MULTI) {
    const int helpers = h->helpers;
    if (helpers > 0 && staged && !b.stats && rows_cap == 4 && per_wave == 64) {
      const size_t lds_h = (size_t)helpers * sink_b + stage_b +
                           ((size_t)helpers * (kHandSlots * (kSlotWords + 1) + 1) + 1) * 4;
      const int64_t blocks = (waves + helpers - 1) / helpers;
      const int64_t blocks_per_cu = (blocks + h->cus - 1) / h->cus;
      if (lds_h <= (size_t)h->lds_limit && (size_t)blocks_per_cu * lds_h <= (size_t)h->lds_per_cu) {
        const dim3 grid_h((unsigned)blocks), block_h((unsigned)(64 * (helpers + 1)));
        const int32_t ww = (int32_t)(sink_b / 4);
#define ASTRA_LAUNCH_HELP(H_)                                                                   \
  do {                                                                                          \
    if (fo.rows)                                                                                \
      hipLaunchKernelGGL((quote_match_kernel<W, false, false, false, true, 4, H_>), grid_h,     \
                         block_h, lds_h, s, b, in, fo, so, steps, budget, ww, per_wave,         \
                         h->hand_lanes, h->hand_queue, h->helper_polls);                         \
    else                                                                                        \
      hipLaunchKernelGGL((quote_match_kernel<W, false, false, false, false, 4, H_>), grid_h,    \
                         block_h, lds_h, s, b, in, fo, so, steps, budget, ww, per_wave,         \
                         h->hand_lanes, h->hand_queue, h->helper_polls);                         \
  } while (0)
        if (helpers == 2)
          ASTRA_LAUNCH_HELP(2);
        else
          ASTRA_LAUNCH_HELP(3);
#undef ASTRA_LAUNCH_HELP
        ASTRA_HIP_CHECK(rt_last_error(), "AddTwoSidedQuotes");
        return ASTRA_OK;
      }
    }
  }
  const size_t wave_bytes = rows_cap == 2 ? sink_b + stage_b : std::max(sink_b, stage_b);
  const size_t lds = (size_t)(h->block / 64) * wave_bytes;
  const int32_t wave_words = (int32_t)(wave_bytes / 4);
  const unsigned grid = grid_for(((int64_t)b.M + per_wave - 1) / per_wave * 64, h->block);
  // (the counting kernels buffer 4 rows whatever the grid: their results are the
  // same, and one depth keeps their number down)
  if (b.stats && fo.rows)
    hipLaunchKernelGGL((quote_match_kernel<W, true, GAME, MULTI, true, 4>), dim3(grid),
                       dim3(h->block), lds, s, b, in, fo, so, steps, budget, wave_words,
                       per_wave, 0, 0, 0);
  else if (b.stats)
    hipLaunchKernelGGL((quote_match_kernel<W, true, GAME, MULTI, false, 4>), dim3(grid),
                       dim3(h->block), lds, s, b, in, fo, so, steps, budget, wave_words,
                       per_wave, 0, 0, 0);
  else if (fo.rows && rows_cap == 2 && !MULTI)
    hipLaunchKernelGGL((quote_match_kernel<W, false, GAME, MULTI, true, MULTI ? 4 : 2>), dim3(grid),
                       dim3(h->block), lds, s, b, in, fo, so, steps, budget, wave_words,
                       per_wave, 0, 0, 0);
  else if (fo.rows)
    hipLaunchKernelGGL((quote_match_kernel<W, false, GAME, MULTI, true, 4>), dim3(grid),
                       dim3(h->block), lds, s, b, in, fo, so, steps, budget, wave_words,
                       per_wave, 0, 0, 0);
  else if (rows_cap == 2 && !MULTI)
    hipLaunchKernelGGL((quote_match_kernel<W, false, GAME, MULTI, false, MULTI ? 4 : 2>), dim3(grid),
                       dim3(h->block), lds, s, b, in, fo, so, steps, budget, wave_words,
                       per_wave, 0, 0, 0);
  else
    hipLaunchKernelGGL((quote_match_kernel<W, false, GAME, MULTI, false, 4>), dim3(grid),
                       dim3(h->block), lds, s, b, in, fo, so, steps, budget, wave_words,
                       per_wave, 0, 0, 0);
#endif
  ASTRA_HIP_CHECK(rt_last_error(), "AddTwoSidedQuotes");
  return ASTRA_OK;
}

int launch_bbo(const astra_market *h, int32_t *bp, int32_t *bs, int32_t *ap, int32_t *as,
               hipStream_t s) {
  const Book b = book_of(h);
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  for (int64_t m = 0; m < b.M; ++m) bbo_copy_market(b, bp, bs, ap, as, m);
#else
  hipLaunchKernelGGL(bbo_kernel, dim3(grid_for(b.M, 256)), dim3(256), 0, s, b, bp, bs, ap, as);
#endif
  ASTRA_HIP_CHECK(rt_last_error(), "GetBBOs");
  return ASTRA_OK;
}

template <int W>
int launch_clear_quotes(const astra_market *h, const uint8_t *reset, hipStream_t s) {
  const Book b = book_of(h);
  const int64_t n = (int64_t)std::max<int32_t>(h->L, 1) * h->M;
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  for (int64_t t = 0; t < n; ++t) clear_quotes_thread<W>(b, reset, t);
#else
  hipLaunchKernelGGL((clear_quotes_kernel<W>), dim3(grid_for(n, 256)), dim3(256), 0, s, b, reset,
                     n);
#endif
  ASTRA_HIP_CHECK(rt_last_error(), "ClearQuotes");
  return ASTRA_OK;
}

template <int W>
int launch_quote_match_plain(const astra_market *h, const QuoteIn &in, const FillOut &fo,
                             hipStream_t s) {
  return launch_quote_match<W, false, false>(h, in, fo, StepOut{}, 1, s);
}

template <int W>
int launch_quote_match_game(const astra_market *h, const QuoteIn &in, const FillOut &fo,
                            hipStream_t s) {
  return launch_quote_match<W, true, false>(h, in, fo, StepOut{}, 1, s);
}

template <int W>
int launch_quote_match_steps(const astra_market *h, const QuoteIn &in, const FillOut &fo,
                             const StepOut &so, int32_t steps, hipStream_t s) {
  return launch_quote_match<W, false, true>(h, in, fo, so, steps, s);
}

#define ASTRA_DISPATCH_W(W_, FN, ...)  \
  switch (W_) {                        \
    case 1: return FN<1>(__VA_ARGS__); \
    case 2: return FN<2>(__VA_ARGS__); \
    case 4: return FN<4>(__VA_ARGS__); \
    case 8: return FN<8>(__VA_ARGS__); \
    default: return FN<16>(__VA_ARGS__); \
  }

int launch_fill(void *dst, int64_t n_words, uint32_t v, hipStream_t s, const char *what) {
  if (n_words <= 0) return ASTRA_OK;
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  uint32_t *d = static_cast<uint32_t *>(dst);
  for (int64_t i = 0; i < n_words; ++i) d[i] = v;
#else
  const int vec = reinterpret_cast<uintptr_t>(dst) % 16 == 0;
  int64_t blocks = ((vec ? n_words / 4 : n_words) + kFillThreads - 1) / kFillThreads;
  blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, 8192));
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(kFillThreads), 0, s,
                     static_cast<uint32_t *>(dst), n_words, v, vec);
#endif
  ASTRA_HIP_CHECK(rt_last_error(), what);
  return ASTRA_OK;
}

int launch_last_price(int32_t *last, const int32_t *counts, const int32_t *prices, int32_t M,
                      int32_t F, int32_t stride, hipStream_t s) {
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  for (int64_t m = 0; m < M; ++m) last_price_market(last, counts, prices, F, stride, m);
#else
  hipLaunchKernelGGL(last_price_kernel, dim3(grid_for(M, 256)), dim3(256), 0, s, last, counts,
                     prices, M, F, stride);
#endif
  ASTRA_HIP_CHECK(rt_last_error(), "UpdateLastPrices");
  return ASTRA_OK;
}

// The TID counter's advance of a call on zero markets, which launches no
// matching kernel (the reference moves its counter on whatever M is).
int advance_tid_empty(astra_market *h, int32_t by, hipStream_t s) {
  int32_t *ctl = reinterpret_cast<int32_t *>(h->ws + h->lay.ctl);
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  ctl[kCtlTid] = (int32_t)((uint32_t)ctl[kCtlTid] + (uint32_t)by);
#else
  hipLaunchKernelGGL(tid_advance_kernel, dim3(1), dim3(64), 0, s, ctl, by);
#endif
  ASTRA_HIP_CHECK(rt_last_error(), "AddTwoSidedQuotes");
  return ASTRA_OK;
}

// Empty book: TID counter 0, masks 0, slot counters 0, BBO cache empty, level
// words NULL, portfolios 0 (the
// order records are left alone: no list reaches a slot before it is written).
int init_book(astra_market *h, hipStream_t s) {
  const Layout &l = h->lay;
  int rc;
  // control words, masks, slot counters and TID counters 0 (market.cu:715)
  if ((rc = launch_fill(h->ws + l.ctl, (int64_t)(l.bbo - l.ctl) / 4, 0u, s, "init"))) return rc;
  // BBO cache of an empty book: both prices NULL
  int32_t *bbo = reinterpret_cast<int32_t *>(h->ws + l.bbo);
  if ((rc = launch_fill(bbo, 2 * (int64_t)h->M, 0xFFFFFFFFu, s, "init"))) return rc;
  if ((rc = launch_fill(h->ws + l.tob, h->M, 0xFFFFFFFFu, s, "init"))) return rc;
  if ((rc = launch_fill(h->ws + l.levels, (int64_t)h->M * h->L * 2, 0xFFFFFFFFu, s, "init")))
    return rc;
  return launch_fill(h->ws + l.portfolios, (int64_t)h->M * h->C * 2, 0u, s, "init");
}

int validate_shape(int32_t M, int32_t L, int32_t O, int32_t F, int32_t C, int32_t flags) {
  const bool ext = (flags & ASTRA_FLAG_EXTENDED_SHAPES) != 0;
  ASTRA_ABI_CHECK(M, >=, 0);
  ASTRA_ABI_CHECK(L, >=, 0);
  ASTRA_ABI_CHECK(O, >=, 1);
  ASTRA_ABI_CHECK(F, >=, 0);
  ASTRA_ABI_CHECK(C, >=, 0);
  ASTRA_ABI_CHECK(M, <=, ASTRA_MAX_MARKETS);
  if (!ext) {  // market.cu:338-342
    ASTRA_ABI_CHECK(L, <=, ASTRA_PRICE_LEVELS);
    ASTRA_ABI_CHECK(O, <=, ASTRA_MAX_ACTIVE_ORDERS_PER_MARKET);
    ASTRA_ABI_CHECK(F, <=, ASTRA_MAX_ACTIVE_FILLS_PER_MARKET);
    ASTRA_ABI_CHECK(C, <=, ASTRA_MAX_CUSTOMERS);
  } else {
    ASTRA_ABI_CHECK(L, <=, ASTRA_EXT_MAX_PRICE_LEVELS);
    ASTRA_ABI_CHECK(O, <=, ASTRA_EXT_MAX_ORDERS);
    ASTRA_ABI_CHECK(F, <=, ASTRA_EXT_MAX_FILLS);
    ASTRA_ABI_CHECK(C, <=, ASTRA_EXT_MAX_CUSTOMERS);
  }
  return ASTRA_OK;
}

int default_stage_budget() {
  const char *e = std::getenv("ASTRA_MARKET_STAGE_BUDGET");
  if (e) {
    const int v = std::atoi(e);
    if (v >= 0) return v;
  }
  return 16;
}

int default_per_wave() {
  const char *e = std::getenv("ASTRA_MARKET_PER_WAVE");
  const int x = e ? std::atoi(e) : 0;
  return (x >= 1 && x <= 64) ? x : 0;
}

// ASTRA_MARKET_FILL_ROWS (2 or 4) fixes the fill rows a lane of the matching
// kernel buffers before writing them out; else fill_rows_per_flush decides.
int32_t default_fill_rows() {
  const char *e = std::getenv("ASTRA_MARKET_FILL_ROWS");
  const int x = e ? std::atoi(e) : 0;
  return (x == 2 || x == 4) ? x : 0;
}

// ASTRA_MARKET_HELPERS: market wavefronts per helper wavefront (2 or 3; 0 turns
// helpers off). ASTRA_MARKET_HAND_LANES: a lane about to walk zero-size orders
// hands its market to the helper when at most this many lanes of its wavefront
// still loop (1-64).
int32_t default_helpers() {
  const char *e = std::getenv("ASTRA_MARKET_HELPERS");
  const int x = e ? std::atoi(e) : 2;
  return (x == 2 || x == 3) ? x : 0;
}

int32_t default_hand_lanes() {
  const char *e = std::getenv("ASTRA_MARKET_HAND_LANES");
  const int x = e ? std::atoi(e) : 64;
  return (x >= 1 && x <= 64) ? x : 64;
}

// ASTRA_MARKET_HAND_QUEUE: markets a helper may hold at once, the one it is
// finishing included (1-13).
int32_t default_hand_queue() {
  const char *e = std::getenv("ASTRA_MARKET_HAND_QUEUE");
  const int x = e ? std::atoi(e) : 2;
  return (x >= 1 && x <= 13) ? x : 2;
}

// ASTRA_MARKET_HELPER_POLLS: idle polls before a helper wavefront gives up
// waiting (at least 1; a small value makes the helpers leave early, which every
// result tolerates: a test knob).
int32_t default_helper_polls() {
  const char *e = std::getenv("ASTRA_MARKET_HELPER_POLLS");
  const int x = e ? std::atoi(e) : 0;
  return x >= 1 ? x : kHelperMaxPolls;
}

int default_block() {
  const char *e = std::getenv("ASTRA_MARKET_BLOCK");
  if (e) {
    const int v = std::atoi(e);
    if (v == 64 || v == 128 || v == 192 || v == 256) return v;
  }
  return 64;  // one wavefront per block: 0.5-3% ahead of 128 on configs 2-4, 256 is worse
}

struct Row {
  int32_t price, size, customer, tid;
};

// Walks one level's list from its head collecting orders with size > 0
// (market.cu:628-642). At most O nodes are visited: the reference loops forever
// on a self-linked slot, which this build does not reproduce.
void walk_level(const std::vector<uint4> &rec, uint32_t head, int32_t price, int32_t O,
                std::vector<Row> &rows) {
  uint32_t slot = head;
  for (int32_t visited = 0; slot < (uint32_t)O && visited < O; ++visited) {
    const uint4 r = rec[slot];
    if ((int32_t)r.x > 0) rows.push_back({price, (int32_t)r.x, (int32_t)r.y, (int32_t)r.z});
    slot = r.w >> 16;
  }
}

}  // namespace

extern "C" {

const char *astra_last_error(void) { return g_last_error.c_str(); }

int astra_market_workspace_size(int32_t M, int32_t L, int32_t O, int32_t F, int32_t C,
                                int32_t flags, size_t *bytes) {
  const int rc = validate_shape(M, L, O, F, C, flags);
  if (rc) return rc;
  if (!bytes) return fail(ASTRA_ERR_INVALID_ARGUMENT, "bytes must not be NULL");
  *bytes = make_layout(M, L, O, C).total;
  return ASTRA_OK;
}

int astra_market_create(int32_t M, int32_t L, int32_t O, int32_t F, int32_t C, int device_id,
                        int32_t threads_per_block, int32_t flags, void *workspace,
                        size_t workspace_bytes, void *stream, astra_market **out) {
  if (!out) return fail(ASTRA_ERR_INVALID_ARGUMENT, "out must not be NULL");
  *out = nullptr;
  int rc = validate_shape(M, L, O, F, C, flags);
  if (rc) return rc;
  ASTRA_ABI_CHECK(threads_per_block, >, 0);  // market.cu:343-344
  ASTRA_ABI_CHECK(threads_per_block, <=, 1024);
  int device_count = 0;
  ASTRA_HIP_CHECK(rt_device_count(&device_count), "hipGetDeviceCount");
  ASTRA_ABI_CHECK(device_id, >=, 0);  // market.cu:349-350
  ASTRA_ABI_CHECK(device_id, <, device_count);
  const Layout lay = make_layout(M, L, O, C);
  if (!workspace && lay.total > 0) return fail(ASTRA_ERR_INVALID_ARGUMENT, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  ASTRA_ABI_CHECK(workspace_bytes, >=, lay.total);
  DeviceGuard g(device_id);
  if (!g.ok) return fail(ASTRA_ERR_HIP, "hipSetDevice failed");
  int lds_limit = 0, lds_per_cu = 0, cus = 0;
  ASTRA_HIP_CHECK(rt_lds_per_block(device_id, &lds_limit), "hipDeviceGetAttribute");
  ASTRA_HIP_CHECK(rt_lds_per_cu(device_id, &lds_per_cu), "hipDeviceGetAttribute");
  ASTRA_HIP_CHECK(rt_cu_count(device_id, &cus), "hipDeviceGetAttribute");
  astra_market *h = new astra_market();
  h->M = M;
  h->L = L;
  h->O = O;
  h->F = F;
  h->C = C;
  h->device = device_id;
  h->threads_per_block = threads_per_block;
  h->flags = flags;
  h->block = default_block();
  h->stage_budget = default_stage_budget();
  h->lds_limit = lds_limit;
  h->lds_per_cu = lds_per_cu > 0 ? lds_per_cu : lds_limit;
  h->cus = cus > 0 ? cus : 1;
  h->per_wave = default_per_wave();
  h->fill_rows = default_fill_rows();
  h->helpers = default_helpers();
  h->hand_lanes = default_hand_lanes();
  h->hand_queue = default_hand_queue();
  h->helper_polls = default_helper_polls();
  h->scratch_word = -1;
  h->stats = nullptr;
  h->ws = static_cast<char *>(workspace);
  h->ws_bytes = workspace_bytes;
  h->lay = lay;
  // the whole workspace to 0 once (order records and alignment padding included, so a
  // fresh workspace holds no garbage), then the empty book's NULL words
  rc = launch_fill(h->ws, (int64_t)(lay.total / 4), 0u, as_stream(stream), "init");
  if (!rc) rc = init_book(h, as_stream(stream));
  if (rc) {
    delete h;
    return rc;
  }
  *out = h;
  return ASTRA_OK;
}

int astra_market_destroy(astra_market *h) {
  if (!h) return ASTRA_OK;
  rt_device_sync(h->device);  // market.cu:416-417
  if (h->scratch_word >= 0) astra_game_release_scratch_word(h->device, h->scratch_word);
  delete h;
  return ASTRA_OK;
}

int astra_market_clone(const astra_market *src, void *dst_ws, size_t dst_bytes, void *stream,
                       astra_market **out) {
  if (!src || !out) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  *out = nullptr;
  ASTRA_ABI_CHECK(dst_bytes, >=, src->lay.total);
  if (!dst_ws && src->lay.total > 0) return fail(ASTRA_ERR_INVALID_ARGUMENT, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(dst_ws) % 256 != 0)
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  DeviceGuard g(src->device);
  if (src->lay.total > 0)
    ASTRA_HIP_CHECK(rt_memcpy(dst_ws, src->ws, src->lay.total, as_stream(stream)), "clone");
  astra_market *h = new astra_market(*src);
  h->stats = nullptr;
  h->scratch_word = -1;  // the copy gets a word of its own on its first such move
  h->ws = static_cast<char *>(dst_ws);
  h->ws_bytes = dst_bytes;
  *out = h;
  return ASTRA_OK;
}

int astra_market_add_two_sided_quotes(astra_market *h, const int32_t *bid_px,
                                      const int32_t *bid_sz, const int32_t *ask_px,
                                      const int32_t *ask_sz, const int32_t *customer_ids,
                                      int32_t *fill_prices, int32_t *fill_sizes,
                                      int32_t *fill_customer_ids, int32_t *fill_quoter_ids,
                                      uint8_t *fill_is_sell_quote, int32_t *fill_quote_sizes,
                                      int32_t *fill_tid, int32_t *fill_quote_tid,
                                      int32_t *fill_counts, void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  if (h->M > 0) {
    if (!bid_px || !bid_sz || !ask_px || !ask_sz || !customer_ids || !fill_counts)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL input or fill_counts pointer");
    if (h->F > 0 && (!fill_prices || !fill_sizes || !fill_customer_ids || !fill_quoter_ids ||
                     !fill_is_sell_quote || !fill_quote_sizes || !fill_tid || !fill_quote_tid))
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL fill pointer");
    DeviceGuard g(h->device);
    const QuoteIn in{bid_px, bid_sz, ask_px, ask_sz, customer_ids};
    const FillOut fo{fill_prices,        fill_sizes,       fill_customer_ids, fill_quoter_ids,
                     fill_is_sell_quote, fill_quote_sizes, fill_tid,          fill_quote_tid,
                     fill_counts,        nullptr};
    // (returns; the kernel moves the TID counter on by 2, market.cu:531)
    ASTRA_DISPATCH_W(h->lay.W, launch_quote_match_plain, h, in, fo, as_stream(stream));
  }
  DeviceGuard g(h->device);
  return advance_tid_empty(h, 2, as_stream(stream));
}

int astra_market_add_two_sided_quotes_rows(astra_market *h, const int32_t *bid_px,
                                           const int32_t *bid_sz, const int32_t *ask_px,
                                           const int32_t *ask_sz, const int32_t *customer_ids,
                                           int32_t *fill_rows, int32_t *fill_counts,
                                           void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  if (h->M > 0) {
    if (!bid_px || !bid_sz || !ask_px || !ask_sz || !customer_ids || !fill_counts)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL input or fill_counts pointer");
    if (h->F > 0 && !fill_rows) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL fill_rows pointer");
    if ((reinterpret_cast<uintptr_t>(fill_rows) & 15) != 0)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "fill_rows must be 16-byte aligned");
    DeviceGuard g(h->device);
    const QuoteIn in{bid_px, bid_sz, ask_px, ask_sz, customer_ids};
    FillOut fo{};
    fo.counts = fill_counts;
    fo.rows = fill_rows;
    // (returns; the kernel moves the TID counter on by 2, market.cu:531)
    ASTRA_DISPATCH_W(h->lay.W, launch_quote_match_plain, h, in, fo, as_stream(stream));
  }
  DeviceGuard g(h->device);
  return advance_tid_empty(h, 2, as_stream(stream));
}

int astra_market_add_two_sided_quotes_steps(
    astra_market *h, int32_t steps, const int32_t *bid_px, const int32_t *bid_sz,
    const int32_t *ask_px, const int32_t *ask_sz, const int32_t *customer_ids,
    int32_t *fill_prices, int32_t *fill_sizes, int32_t *fill_customer_ids, int32_t *fill_quoter_ids,
    uint8_t *fill_is_sell_quote, int32_t *fill_quote_sizes, int32_t *fill_tid,
    int32_t *fill_quote_tid, int32_t *fill_rows, int32_t *fill_counts, int32_t *step_fill_counts,
    int32_t *step_bbos, void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  if (steps < 0) return fail(ASTRA_ERR_INVALID_ARGUMENT, "steps must be >= 0");
  if (steps == 0) return ASTRA_OK;
  if (h->M > 0) {
    if (!bid_px || !bid_sz || !ask_px || !ask_sz || !customer_ids || !fill_counts)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL input or fill_counts pointer");
    if (fill_rows) {
      if ((reinterpret_cast<uintptr_t>(fill_rows) & 15) != 0)
        return fail(ASTRA_ERR_INVALID_ARGUMENT, "fill_rows must be 16-byte aligned");
    } else if (h->F > 0 && (!fill_prices || !fill_sizes || !fill_customer_ids || !fill_quoter_ids ||
                            !fill_is_sell_quote || !fill_quote_sizes || !fill_tid ||
                            !fill_quote_tid)) {
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL fill pointer");
    }
    DeviceGuard g(h->device);
    const QuoteIn in{bid_px, bid_sz, ask_px, ask_sz, customer_ids};
    FillOut fo{};
    fo.counts = fill_counts;
    if (fill_rows) {
      fo.rows = fill_rows;
    } else {
      fo = FillOut{fill_prices,        fill_sizes,       fill_customer_ids, fill_quoter_ids,
                   fill_is_sell_quote, fill_quote_sizes, fill_tid,          fill_quote_tid,
                   fill_counts,        nullptr};
    }
    StepOut so{};
    so.counts = step_fill_counts;
    so.bbo[0] = step_bbos;  // step_views derives the other three fields' rows
    // (returns; the kernel moves the TID counter on by 2 per step, market.cu:531)
    ASTRA_DISPATCH_W(h->lay.W, launch_quote_match_steps, h, in, fo, so, steps, as_stream(stream));
  }
  DeviceGuard g(h->device);
  return advance_tid_empty(h, (int32_t)(2u * (uint32_t)steps), as_stream(stream));
}

}  // extern "C"

int astra_game_device(const astra_market *h) { return h ? h->device : 0; }
int astra_game_scratch_word(const astra_market *h) { return h->scratch_word; }
void astra_game_set_scratch_word(astra_market *h, int word) { h->scratch_word = word; }

int astra_game_move(astra_market *h, const GameMove &g, int32_t *const fill_fields[8],
                    int32_t *fill_rows, int32_t *fill_counts, hipStream_t stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  if (h->M > 0) {
    DeviceGuard dg(h->device);
    QuoteIn in{nullptr, nullptr, nullptr, nullptr, nullptr, g};
    if ((reinterpret_cast<uintptr_t>(fill_rows) & 15) != 0)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "fill_rows must be 16-byte aligned");
    FillOut fo{};
    fo.counts = fill_counts;
    if (fill_rows) {
      fo.rows = fill_rows;
    } else {
      fo.prices = fill_fields[0];
      fo.sizes = fill_fields[1];
      fo.taker = fill_fields[2];
      fo.quoter = fill_fields[3];
      fo.is_sell_quote = reinterpret_cast<uint8_t *>(fill_fields[4]);
      fo.quote_sizes = fill_fields[5];
      fo.tid = fill_fields[6];
      fo.quote_tid = fill_fields[7];
    }
    // (returns; the kernel moves the TID counter on by 2, market.cu:531,
    // unless the move's checks failed)
    ASTRA_DISPATCH_W(h->lay.W, launch_quote_match_game, h, in, fo, stream);
  }
  DeviceGuard dg(h->device);
  return advance_tid_empty(h, 2, stream);
}

extern "C" {

int astra_market_get_bbos(const astra_market *h, int32_t *bid_px, int32_t *bid_sz,
                          int32_t *ask_px, int32_t *ask_sz, void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  if (h->M == 0) return ASTRA_OK;
  if (!bid_px || !bid_sz || !ask_px || !ask_sz)
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL BBO pointer");
  DeviceGuard g(h->device);
  return launch_bbo(h, bid_px, bid_sz, ask_px, ask_sz, as_stream(stream));
}

int astra_update_last_prices(int32_t *last, const int32_t *counts, const int32_t *prices,
                             int32_t M, int32_t F, void *stream) {
  ASTRA_ABI_CHECK(M, >=, 0);
  ASTRA_ABI_CHECK(F, >=, 0);
  if (M == 0) return ASTRA_OK;
  if (!last || !counts || (F > 0 && !prices))
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL pointer");
  return launch_last_price(last, counts, prices, M, F, 1, as_stream(stream));
}

int astra_update_last_prices_rows(int32_t *last, const int32_t *counts, const int32_t *fill_rows,
                                  int32_t M, int32_t F, void *stream) {
  ASTRA_ABI_CHECK(M, >=, 0);
  ASTRA_ABI_CHECK(F, >=, 0);
  if (M == 0) return ASTRA_OK;
  if (!last || !counts || (F > 0 && !fill_rows))
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL pointer");
  return launch_last_price(last, counts, fill_rows, M, F, 8, as_stream(stream));
}

int astra_fill_i32(int32_t *dst, int64_t count, int32_t value, void *stream) {
  ASTRA_ABI_CHECK(count, >=, 0);
  if (count == 0) return ASTRA_OK;
  if (!dst) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL pointer");
  return launch_fill(dst, count, (uint32_t)value, as_stream(stream), "fill");
}

int astra_market_reset(astra_market *h, void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  DeviceGuard g(h->device);
  return init_book(h, as_stream(stream));  // market.cu:699-715, the TID counter included
}

int astra_market_clear_quotes(astra_market *h, const uint8_t *reset, void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  if (h->M == 0) return ASTRA_OK;
  if (!reset) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL reset mask");
  DeviceGuard g(h->device);
  ASTRA_DISPATCH_W(h->lay.W, launch_clear_quotes, h, reset, as_stream(stream));
}

int astra_market_portfolios(const astra_market *h, int32_t **p) {
  if (!h || !p) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL argument");
  *p = reinterpret_cast<int32_t *>(h->ws + h->lay.portfolios);
  return ASTRA_OK;
}

int astra_market_shape(const astra_market *h, int32_t *M, int32_t *L, int32_t *O, int32_t *F,
                       int32_t *C) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_market_shape: null handle");
  if (M) *M = h->M;
  if (L) *L = h->L;
  if (O) *O = h->O;
  if (F) *F = h->F;
  if (C) *C = h->C;
  return ASTRA_OK;
}

int astra_market_to_string(const astra_market *h, int32_t market_id, char *buf, size_t buflen,
                           size_t *needed, void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  std::string s;
  char line[160];
  if (market_id >= h->M || market_id < 0) {  // market.cu:602-604
    std::snprintf(line, sizeof line, "Error: Invalid market_id %d (num_markets = %d)", market_id,
                  h->M);
    s = line;
  } else {
    DeviceGuard g(h->device);
    std::vector<uint16_t> lv((size_t)h->L * 4);
    std::vector<uint4> rec((size_t)h->O);
    hipStream_t st = as_stream(stream);
    if (h->L > 0)
      ASTRA_HIP_CHECK(rt_memcpy(lv.data(), h->ws + h->lay.levels + (size_t)market_id * h->L * 8,
                                (size_t)h->L * 8, st),
                      "ToString");
    ASTRA_HIP_CHECK(rt_memcpy(rec.data(), h->ws + h->lay.records + (size_t)market_id * h->O * 16,
                              (size_t)h->O * 16, st),
                    "ToString");
    ASTRA_HIP_CHECK(rt_sync(st), "ToString");
    std::vector<Row> sells, buys;
    for (int32_t p = 0; p < h->L; ++p) walk_level(rec, lv[(size_t)p * 4 + 2], p, h->O, sells);
    std::sort(sells.begin(), sells.end(), [](const Row &a, const Row &b) {  // :645-651
      if (a.price != b.price) return a.price > b.price;
      return a.tid < b.tid;
    });
    for (int32_t p = h->L - 1; p >= 0; --p) walk_level(rec, lv[(size_t)p * 4], p, h->O, buys);
    std::snprintf(line, sizeof line, "####### %zu sell orders #######\n", sells.size());  // :677
    s += line;
    for (const Row &r : sells) {
      std::snprintf(line, sizeof line, "px %d @ sz %d   id=%d @ t=%d\n", r.price, r.size,
                    r.customer, r.tid);
      s += line;
    }
    s += "#############################\n";
    std::snprintf(line, sizeof line, "####### %zu buy orders #######\n", buys.size());
    s += line;
    for (const Row &r : buys) {
      std::snprintf(line, sizeof line, "px %d @ sz %d   id=%d @ t=%d\n", r.price, r.size,
                    r.customer, r.tid);
      s += line;
    }
    s += "#############################";
  }
  if (needed) *needed = s.size();
  if (buf && buflen > 0) {
    const size_t k = std::min(buflen - 1, s.size());
    std::memcpy(buf, s.data(), k);
    buf[k] = '\0';
  }
  return ASTRA_OK;
}

int astra_market_set_stats(astra_market *h, int64_t *counters) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  if (reinterpret_cast<uintptr_t>(counters) % 8 != 0)
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "counters must be 8-byte aligned");
  h->stats = reinterpret_cast<unsigned long long *>(counters);
  return ASTRA_OK;
}

int astra_market_get_tid(const astra_market *h, int32_t *tid, void *stream) {
  if (!h || !tid) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL argument");
  DeviceGuard g(h->device);
  hipStream_t st = as_stream(stream);
  // every market's copy holds the counter; a market-less book keeps it in ctl
  const char *src = h->M > 0 ? h->ws + h->lay.tids : h->ws + h->lay.ctl + kCtlTid * 4;
  ASTRA_HIP_CHECK(rt_memcpy(tid, src, sizeof(int32_t), st), "get_tid");
  ASTRA_HIP_CHECK(rt_sync(st), "get_tid");
  return ASTRA_OK;
}

int astra_market_set_tid(astra_market *h, int32_t tid, void *stream) {
  if (!h) return fail(ASTRA_ERR_INVALID_ARGUMENT, "NULL handle");
  DeviceGuard g(h->device);
  const int rc = launch_fill(h->ws + h->lay.ctl + kCtlTid * 4, 1, (uint32_t)tid, as_stream(stream),
                             "set_tid");
  if (rc) return rc;
  return launch_fill(h->ws + h->lay.tids, h->M, (uint32_t)tid, as_stream(stream), "set_tid");
}

}  // extern "C"

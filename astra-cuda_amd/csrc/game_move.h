// game_move.h -- the high-low game's trading move fused into the matching
// kernel (nlyu1/astra-cuda src/games/high_low_trading/high_low_trading.cc:247-329).
//
// One lane per env does, around its market's matching: before it, the range
// checks of the move (:264-271; a bit per failed check is OR-ed into *errors)
// and the snapshot of the players' portfolios (CopyCustomerPortfoliosTo, :257);
// after it, GetBBOs and UpdateLastPrices (:279-280), the telemetry rows
// (:284-288) and every player's immediate reward and reward since last action
// (:277, :290-328) in int32 with wrap-around, as libtorch's int32 kernels do.
// The matching kernel's own inputs come from the move row (:260-263) and the
// acting player (the customer id, :264).
#pragma once

#include <cstdint>

struct astra_market;

struct GameMove {
  const int32_t *move;          // [M,4]: bid_px, ask_px, bid_sz, ask_sz
  int32_t *last_pos;            // [M,P,2]
  const int32_t *target;        // [M,P]
  const int32_t *contract_values;  // [M,3]
  int32_t *pcot;                // [T,P,6,M]: env-minor, word (m,p,t,f) at ((t*P+p)*6+f)*M+m
                                // (M = the market's env count)
  int32_t *mcot;                // [P*T,3,M]: env-minor, word (m,k,f) at (k*3+f)*M+m
  int32_t *imm, *rsla;          // [M,P]
  int32_t *bbo_out[4];          // best bid px, bid size, ask px, ask size [M]
  int32_t *last_prices;         // [M]
  int32_t *errors;              // [1]
  int32_t P, T, S, V, player, tmn;
  int32_t abort_on_error;       // 1: *errors != 0 (set by the checks launched
                                // before) makes every env leave all state as is
};

// The move's four values and the range-check bits (high_low_trading.cc:264-271).
struct GameQuote {
  int32_t bid_px, ask_px, bid_sz, ask_sz, bad;
};

ASTRA_HD GameQuote game_quote(const GameMove &g, int64_t m) {
  GameQuote q;
  q.bid_px = g.move[m * 4 + 0];
  q.ask_px = g.move[m * 4 + 1];
  q.bid_sz = g.move[m * 4 + 2];
  q.ask_sz = g.move[m * 4 + 3];
  q.bad = (!(q.bid_px > 0) ? 1 : 0) | (!(q.ask_px > 0) ? 2 : 0) | (!(q.bid_px <= g.V) ? 4 : 0) |
          (!(q.ask_px <= g.V) ? 8 : 0) | (!(q.bid_sz >= 0) ? 16 : 0) | (!(q.ask_sz >= 0) ? 32 : 0) |
          (!(q.bid_sz <= g.S) ? 64 : 0) | (!(q.ask_sz <= g.S) ? 128 : 0);
  return q;
}

ASTRA_HD int32_t g_add(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
ASTRA_HD int32_t g_sub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
ASTRA_HD int32_t g_mul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
ASTRA_HD int32_t g_abs(int32_t a) { return a < 0 ? (int32_t)(0u - (uint32_t)a) : a; }

// Loads a portfolio word past the L1 cache: the lane's own fire-and-forget
// atomics updated it at L2 after an earlier read may have cached it in L1.
ASTRA_HD int32_t load_past_l1(const int32_t *p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#else
  return *p;
#endif
}

// Players are handled kPlayerBatch at a time, every load of a batch issued
// before any of its stores: the compiler cannot tell the arrays apart, so a
// load placed after a store waits for the store, one round trip per load. The
// loads are unconditional (a batch slot beyond the last player reads the last
// player again): a load under a branch is waited for where the branch ends.
constexpr int32_t kPlayerBatch = 8;

// The portfolios of env m's first kPlayerBatch players, loaded for the
// snapshot game_before stores; loaded together with the market's first words,
// so the snapshot takes no round trip of its own.
struct GameSnap {
  int32_t con[kPlayerBatch], cash[kPlayerBatch];
};

ASTRA_HD GameSnap game_snapshot(const GameMove &g, const int32_t *pf_m) {
  GameSnap s;
#pragma unroll
  for (int32_t j = 0; j < kPlayerBatch; ++j) {
    const int32_t q = j < g.P ? j : g.P - 1;
    s.con[j] = pf_m[q * 2];
    s.cash[j] = pf_m[q * 2 + 1];
  }
  return s;
}

// Before the matching: the check bits and the portfolio snapshot
// (CopyCustomerPortfoliosTo, :257) of env m.
ASTRA_HD void game_before(const GameMove &g, const GameSnap &snap, const int32_t *pf_m, int64_t m,
                          int32_t bad) {
  if (bad) {
#if defined(__HIP_DEVICE_COMPILE__)
    atomicOr(g.errors, bad);
#else
    *g.errors |= bad;
#endif
  }
  int32_t *last = g.last_pos + m * g.P * 2;
#pragma unroll
  for (int32_t j = 0; j < kPlayerBatch; ++j) {
    if (j < g.P) {
      last[j * 2] = snap.con[j];
      last[j * 2 + 1] = snap.cash[j];
    }
  }
  for (int32_t p0 = kPlayerBatch; p0 < g.P; p0 += kPlayerBatch) {
    int32_t con[kPlayerBatch], cash[kPlayerBatch];
#pragma unroll
    for (int32_t j = 0; j < kPlayerBatch; ++j) {
      const int32_t q = p0 + j < g.P ? p0 + j : g.P - 1;
      con[j] = pf_m[q * 2];
      cash[j] = pf_m[q * 2 + 1];
    }
#pragma unroll
    for (int32_t j = 0; j < kPlayerBatch; ++j) {
      if (p0 + j < g.P) {
        last[(p0 + j) * 2] = con[j];
        last[(p0 + j) * 2 + 1] = cash[j];
      }
    }
  }
}

// After the matching (its fill rows and portfolio atomics issued): BBO, last
// price, telemetry and rewards of env m of M. fills = this call's fill count,
// last_px = the price of its last fill row.
ASTRA_HD void game_after(const GameMove &g, const GameQuote &q, const int32_t *pf_m, int64_t M,
                         int64_t m, const int32_t (&bbo)[4], int32_t fills, int32_t last_px) {
  for (int k = 0; k < 4; ++k) g.bbo_out[k][m] = bbo[k];
  int32_t last = g.last_prices[m];
  if (fills > 0) {  // UpdateLastPrices (market.cu:767-786)
    last = last_px;
    g.last_prices[m] = last;
  }
  const int32_t P = g.P, T = g.T, V = g.V, player = g.player, tmn = g.tmn, pmn = tmn / P;
  // this round's rows of env m: word (p, f) at (p*6+f)*M, so a wavefront's lanes
  // store consecutive words
  int32_t *pc = g.pcot + (int64_t)pmn * P * 6 * M + m;
  int32_t *mine = pc + (int64_t)player * 6 * M;
  mine[0] = q.bid_px;
  mine[M] = q.ask_px;
  mine[2 * M] = q.bid_sz;
  mine[3 * M] = q.ask_sz;
  int32_t *mc = g.mcot + (int64_t)tmn * 3 * M + m;
  mc[0] = bbo[0];
  mc[M] = bbo[2];
  mc[2 * M] = last;
  const int32_t mn = q.bid_sz < q.ask_sz ? q.bid_sz : q.ask_sz;
  const int32_t cross = g_add(g_sub(q.bid_px, q.ask_px), 1);
  const int32_t penalty = g_mul(g_mul(g_add(mn, 1), cross > 0 ? cross : 0), V);  // :308
  const int32_t bid_cheap = (q.bid_sz == 0 && q.bid_px != 1) ? V : 0;          // :314
  const int32_t ask_cheap = (q.ask_sz == 0 && q.ask_px != V) ? V : 0;          // :315
  const bool settle = tmn == T * P - 1;                                         // :319
  const int32_t value = g.contract_values[m * 3 + 2];
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_s_waitcnt(0);  // this lane's portfolio atomics have reached L2
#endif
  for (int32_t p0 = 0; p0 < P; p0 += kPlayerBatch) {
    int32_t c_con[kPlayerBatch], c_cash[kPlayerBatch], l_con[kPlayerBatch], l_cash[kPlayerBatch];
    int32_t tgt[kPlayerBatch], since[kPlayerBatch];
#pragma unroll
    for (int32_t j = 0; j < kPlayerBatch; ++j) {
      const int32_t q = p0 + j < P ? p0 + j : P - 1;
      c_con[j] = load_past_l1(pf_m + q * 2);
      c_cash[j] = load_past_l1(pf_m + q * 2 + 1);
      l_con[j] = g.last_pos[(m * P + q) * 2];
      l_cash[j] = g.last_pos[(m * P + q) * 2 + 1];
      tgt[j] = g.target[m * P + q];
      since[j] = g.rsla[m * P + q];
    }
#pragma unroll
    for (int32_t j = 0; j < kPlayerBatch; ++j) {
      const int32_t p = p0 + j;
      if (p < P) {
        pc[((int64_t)p * 6 + 4) * M] = c_con[j];
        pc[((int64_t)p * 6 + 5) * M] = c_cash[j];
        int32_t r = tgt[j] != 0
                        ? g_mul(g_sub(g_abs(g_sub(l_con[j], tgt[j])), g_abs(g_sub(c_con[j], tgt[j]))), V)
                        : 0;
        r = g_add(r, g_sub(c_cash[j], l_cash[j]));
        if (p == player) r = g_sub(g_sub(g_sub(r, penalty), bid_cheap), ask_cheap);
        if (settle) r = g_add(r, g_mul(c_con[j], value));
        g.imm[m * P + p] = r;
        const int32_t before = p == player ? 0 : since[j];  // :277
        g.rsla[m * P + p] = g_add(before, r);
      }
    }
  }
}

// One fused trading move of every env of `market` (implemented with the matching
// kernel in market.hip): the fills go to the [M,F,8] rows when `fill_rows` is set,
// else to the eight field arrays; advances the TID counter by 2 like
// astra_market_add_two_sided_quotes.
int astra_game_move(astra_market *market, const GameMove &g, int32_t *const fill_fields[8],
                    int32_t *fill_rows, int32_t *fill_counts, hipStream_t stream);

// The device the market lives on.
int astra_game_device(const astra_market *market);

// The word of the library's per-device scratch that the market's allocation-free
// moves use (-1 until its first such move), its assignment, and the release of a
// word when its market is destroyed (implemented in high_low.hip).
int astra_game_scratch_word(const astra_market *market);
void astra_game_set_scratch_word(astra_market *market, int word);
void astra_game_release_scratch_word(int device, int word);

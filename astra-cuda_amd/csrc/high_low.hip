// high_low.hip -- the high-low trading game's per-move kernels (MI355X, gfx950)
// behind the C ABI of include/astra_high_low.h.
//
// Semantics follow nlyu1/astra-cuda src/games/high_low_trading/high_low_trading.cc:
// the trading move HighLowTradingState::ApplyPlayerTrading (:247-329) and
// FillObservationTensor (:510-602). The reference spreads a move over about forty
// libtorch launches and eight .item() syncs; here it is
//
//   1. trade_pre_kernel: one lane per env checks the move against the
//      reference's ranges (OR-ing a bit per failed check into *errors), splits
//      the [N,4] move into the matching kernel's input columns, writes the
//      customer id (the acting player), and snapshots the env's portfolios into
//      player_last_positions (CopyCustomerPortfoliosTo, :257);
//   2. the VecMarket matching kernel (astra_market_add_two_sided_quotes);
//   3. trade_post_kernel: one lane per env copies the BBO the matching kernel
//      left (GetBBOs), updates the last price (UpdateLastPrices), writes the
//      telemetry rows and computes every player's immediate reward and reward
//      since last action (:280-328) in int32 with wrap-around, as libtorch's
//      int32 kernels do.
//
// With check = 1 the host waits once after step 1 and stops with an error, like
// the reference's checks, before anything trades; with check = 0 nothing waits.
//
// The kernel bodies are __host__ __device__ functions; the host-emulation build
// (-DASTRA_HOST_EMULATION) runs them as loops over host memory.
#include <cmath>
#include <string>

#include "astra_high_low.h"

#define ASTRA_SRC_NAME "high_low.hip"
#include "runtime.h"

using namespace astra_rt;

namespace {

constexpr int kBlock = 256;

ASTRA_HD int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
ASTRA_HD int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
ASTRA_HD int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
ASTRA_HD int32_t wabs(int32_t a) { return a < 0 ? (int32_t)(0u - (uint32_t)a) : a; }  // abs(INT_MIN) stays

struct TradeArgs {
  astra_hl_trade t;
  const int32_t *portfolios;  // [N,C,2]
  const int32_t *bbo_cache;   // [4,N]
  int32_t N, C, F;
};

// Step 1 for env n.
ASTRA_HD void trade_pre(const TradeArgs &a, int64_t n) {
  const astra_hl_trade &t = a.t;
  const int64_t N = a.N;
  const int32_t bid_px = t.move[n * 4 + 0], ask_px = t.move[n * 4 + 1];
  const int32_t bid_sz = t.move[n * 4 + 2], ask_sz = t.move[n * 4 + 3];
  const int32_t V = t.max_contract_value, S = t.max_contracts_per_trade;
  int32_t bad = 0;  // high_low_trading.cc:264-271, in order
  if (!(bid_px > 0)) bad |= ASTRA_HL_ERR_BID_PRICE_LOW;
  if (!(ask_px > 0)) bad |= ASTRA_HL_ERR_ASK_PRICE_LOW;
  if (!(bid_px <= V)) bad |= ASTRA_HL_ERR_BID_PRICE_HIGH;
  if (!(ask_px <= V)) bad |= ASTRA_HL_ERR_ASK_PRICE_HIGH;
  if (!(bid_sz >= 0)) bad |= ASTRA_HL_ERR_BID_SIZE_LOW;
  if (!(ask_sz >= 0)) bad |= ASTRA_HL_ERR_ASK_SIZE_LOW;
  if (!(bid_sz <= S)) bad |= ASTRA_HL_ERR_BID_SIZE_HIGH;
  if (!(ask_sz <= S)) bad |= ASTRA_HL_ERR_ASK_SIZE_HIGH;
  if (bad) {
#if defined(__HIP_DEVICE_COMPILE__)
    atomicOr(t.errors, bad);
#else
    *t.errors |= bad;
#endif
  }
  t.columns[n] = bid_px;
  t.columns[N + n] = bid_sz;
  t.columns[2 * N + n] = ask_px;
  t.columns[3 * N + n] = ask_sz;
  t.columns[4 * N + n] = t.player;
  const int32_t P = t.players;
  for (int32_t p = 0; p < P; ++p) {
    t.player_last_positions[(n * P + p) * 2] = a.portfolios[(n * a.C + p) * 2];
    t.player_last_positions[(n * P + p) * 2 + 1] = a.portfolios[(n * a.C + p) * 2 + 1];
  }
}

// Step 3 for env n.
ASTRA_HD void trade_post(const TradeArgs &a, int64_t n) {
  const astra_hl_trade &t = a.t;
  const int64_t N = a.N;
  const int32_t P = t.players, T = t.steps_per_player, V = t.max_contract_value;
  const int32_t player = t.player, tmn = t.trade_move_number, pmn = tmn / P;
  // GetBBOs (:279) and UpdateLastPrices (:280, market.cu:767-786)
  const int32_t bbp = a.bbo_cache[n], bbs = a.bbo_cache[N + n];
  const int32_t bap = a.bbo_cache[2 * N + n], bas = a.bbo_cache[3 * N + n];
  t.best_bid_prices[n] = bbp;
  t.best_bid_sizes[n] = bbs;
  t.best_ask_prices[n] = bap;
  t.best_ask_sizes[n] = bas;
  const int32_t cnt = t.fill_counts[n];
  int32_t last = t.last_prices[n];
  if (cnt > 0 && cnt <= a.F) {
    last = t.fill_rows ? t.fill_rows[(n * a.F + (cnt - 1)) * 8] : t.fill_prices[n * a.F + (cnt - 1)];
    t.last_prices[n] = last;
  }
  // telemetry (:284-288)
  const int32_t bid_px = t.move[n * 4 + 0], ask_px = t.move[n * 4 + 1];
  const int32_t bid_sz = t.move[n * 4 + 2], ask_sz = t.move[n * 4 + 3];
  int32_t *pc = t.player_contract_over_time + (n * P) * T * 6;
  int32_t *mine = pc + ((int64_t)player * T + pmn) * 6;
  mine[0] = bid_px;
  mine[1] = ask_px;
  mine[2] = bid_sz;
  mine[3] = ask_sz;
  int32_t *mc = t.market_contract_over_time + (n * (int64_t)P * T + tmn) * 3;
  mc[0] = bbp;
  mc[1] = bap;
  mc[2] = last;
  // rewards (:290-328)
  const int32_t mn = bid_sz < ask_sz ? bid_sz : ask_sz;
  const int32_t cross = wadd(wsub(bid_px, ask_px), 1);
  const int32_t penalty =
      wmul(wmul(wadd(mn, 1), cross > 0 ? cross : 0), V);                              // :308
  const int32_t bid_cheap = (bid_sz == 0 && bid_px != 1) ? V : 0;                     // :314
  const int32_t ask_cheap = (ask_sz == 0 && ask_px != V) ? V : 0;                     // :315
  const bool settle = tmn == T * P - 1;                                                 // :319
  const int32_t value = t.contract_values[n * 3 + 2];
  for (int32_t p = 0; p < P; ++p) {
    const int32_t c_con = a.portfolios[(n * a.C + p) * 2];
    const int32_t c_cash = a.portfolios[(n * a.C + p) * 2 + 1];
    const int32_t l_con = t.player_last_positions[(n * P + p) * 2];
    const int32_t l_cash = t.player_last_positions[(n * P + p) * 2 + 1];
    const int32_t tgt = t.target_positions[n * P + p];
    pc[((int64_t)p * T + pmn) * 6 + 4] = c_con;
    pc[((int64_t)p * T + pmn) * 6 + 5] = c_cash;
    const int32_t prev_diff = wabs(wsub(l_con, tgt)), cur_diff = wabs(wsub(c_con, tgt));
    int32_t r = tgt != 0 ? wmul(wsub(prev_diff, cur_diff), V) : 0;
    r = wadd(r, wsub(c_cash, l_cash));
    if (p == player) r = wsub(wsub(wsub(r, penalty), bid_cheap), ask_cheap);
    if (settle) r = wadd(r, wmul(c_con, value));
    t.immediate_rewards[n * P + p] = r;
    const int32_t before = p == player ? 0 : t.rewards_since_last_action[n * P + p];  // :277
    t.rewards_since_last_action[n * P + p] = wadd(before, r);
  }
}

// One element of the [N, 6 + 1 + 6P + 5] observation (:510-602).
ASTRA_HD void observation_element(const astra_hl_observation &o, int64_t i) {
  const int32_t P = o.players, T = o.steps_per_player, player = o.player, cr = o.current_round;
  const int64_t D = 6 + 1 + 6 * (int64_t)P + 5;
  const int64_t n = i / D;
  const int32_t j = (int32_t)(i - n * D);
  const int32_t perm = o.player_permutation[n * P + player];
  float v = 0.0f;
  if (j == 0) {
    v = (perm == 0 || perm == 1) ? 1.0f : 0.0f;
  } else if (j == 1) {
    v = perm == 2 ? 1.0f : 0.0f;
  } else if (j == 2) {
    v = perm > 2 ? 1.0f : 0.0f;
  } else if (j == 3) {
    v = o.player_sin;
  } else if (j == 4) {
    v = o.player_cos;
  } else if (j == 5) {  // private information (:536-546)
    if (perm == 0) v = (float)o.contract_values[n * 3];
    else if (perm == 1) v = (float)o.contract_values[n * 3 + 1];
    else if (perm == 2) v = o.contract_high_settle[n] ? 1.0f : 0.0f;
    else if (perm > 2) v = (float)o.target_positions[n * P + player];
  } else if (j == 6) {
    v = o.round_fraction;
  } else if (j < 7 + 6 * P) {  // the rounds of player_contract_over_time (:559-584)
    const int32_t q = j - 7, p = q / 6, f = q - 6 * (q / 6);
    int32_t r;
    if (cr == 0 || player == P - 1) r = cr;
    else if (player == 0) r = cr - 1;
    else r = p < player ? cr : cr - 1;
    v = (float)o.player_contract_over_time[((n * P + p) * T + r) * 6 + f];
  } else {  // BBO and last price (:589-599)
    const int32_t k = j - (7 + 6 * P);
    const int32_t *src = k == 0   ? o.best_bid_prices
                         : k == 1 ? o.best_ask_prices
                         : k == 2 ? o.best_bid_sizes
                         : k == 3 ? o.best_ask_sizes
                                  : o.last_prices;
    v = (float)src[n];
  }
  o.values[i] = v;
}

__global__ __launch_bounds__(kBlock) void trade_pre_kernel(TradeArgs a) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n < a.N) trade_pre(a, n);
}

__global__ __launch_bounds__(kBlock) void trade_post_kernel(TradeArgs a) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n < a.N) trade_post(a, n);
}

__global__ __launch_bounds__(kBlock) void observation_kernel(astra_hl_observation o, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < total) observation_element(o, i);
}

inline unsigned grid_for(int64_t n) { return (unsigned)((n + kBlock - 1) / kBlock); }

int launch_pre(const TradeArgs &a, hipStream_t s) {
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  for (int64_t n = 0; n < a.N; ++n) trade_pre(a, n);
  return ASTRA_OK;
#else
  if (a.N > 0) hipLaunchKernelGGL(trade_pre_kernel, dim3(grid_for(a.N)), dim3(kBlock), 0, s, a);
  ASTRA_HIP_CHECK(rt_last_error(), "trade_pre_kernel launch");
  return ASTRA_OK;
#endif
}

int launch_post(const TradeArgs &a, hipStream_t s) {
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  for (int64_t n = 0; n < a.N; ++n) trade_post(a, n);
  return ASTRA_OK;
#else
  if (a.N > 0) hipLaunchKernelGGL(trade_post_kernel, dim3(grid_for(a.N)), dim3(kBlock), 0, s, a);
  ASTRA_HIP_CHECK(rt_last_error(), "trade_post_kernel launch");
  return ASTRA_OK;
#endif
}

const char *check_text(int32_t bits) {  // the first failed check, as the reference would stop
  if (bits & ASTRA_HL_ERR_BID_PRICE_LOW) return "torch::min(bid_prices).item<int>() > 0";
  if (bits & ASTRA_HL_ERR_ASK_PRICE_LOW) return "torch::min(ask_prices).item<int>() > 0";
  if (bits & ASTRA_HL_ERR_BID_PRICE_HIGH)
    return "torch::max(bid_prices).item<int>() <= GetGame()->GetMaxContractValue()";
  if (bits & ASTRA_HL_ERR_ASK_PRICE_HIGH)
    return "torch::max(ask_prices).item<int>() <= GetGame()->GetMaxContractValue()";
  if (bits & ASTRA_HL_ERR_BID_SIZE_LOW) return "torch::min(bid_sizes).item<int>() >= 0";
  if (bits & ASTRA_HL_ERR_ASK_SIZE_LOW) return "torch::min(ask_sizes).item<int>() >= 0";
  if (bits & ASTRA_HL_ERR_BID_SIZE_HIGH)
    return "torch::max(bid_sizes).item<int>() <= GetGame()->GetMaxContractsPerTrade()";
  return "torch::max(ask_sizes).item<int>() <= GetGame()->GetMaxContractsPerTrade()";
}

}  // namespace

extern "C" {

int astra_high_low_trade(astra_market *market, const astra_hl_trade *t, void *stream) {
  ASTRA_ABI_CHECK(market != nullptr, ==, true);
  ASTRA_ABI_CHECK(t != nullptr, ==, true);
  int32_t M = 0, L = 0, O = 0, F = 0, C = 0;
  int rc = astra_market_shape(market, &M, &L, &O, &F, &C);
  if (rc) return rc;
  ASTRA_ABI_CHECK(t->players, >=, 1);
  ASTRA_ABI_CHECK(t->players, <=, C);
  ASTRA_ABI_CHECK(t->steps_per_player, >=, 1);
  ASTRA_ABI_CHECK(t->player, >=, 0);
  ASTRA_ABI_CHECK(t->player, <, t->players);
  ASTRA_ABI_CHECK(t->trade_move_number, >=, 0);  // :251-253
  ASTRA_ABI_CHECK(t->trade_move_number, <, (int64_t)t->steps_per_player * t->players);
  ASTRA_ABI_CHECK(t->trade_move_number % t->players, ==, t->player);
  const void *need[] = {t->move, t->columns, t->player_last_positions, t->target_positions,
                        t->contract_values, t->player_contract_over_time,
                        t->market_contract_over_time, t->immediate_rewards,
                        t->rewards_since_last_action, t->fill_counts, t->best_bid_prices,
                        t->best_bid_sizes, t->best_ask_prices, t->best_ask_sizes,
                        t->last_prices, t->errors};
  for (const void *p : need)
    if (M > 0 && p == nullptr)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_high_low_trade: null pointer in astra_hl_trade");
  const void *fields[] = {t->fill_prices, t->fill_sizes, t->fill_customer_ids, t->fill_quoter_ids,
                          t->fill_is_sell_quote, t->fill_quote_sizes, t->fill_tid,
                          t->fill_quote_tid};
  if (!t->fill_rows)
    for (const void *p : fields)
      if (M > 0 && p == nullptr)
        return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_high_low_trade: null fill pointer");
  TradeArgs a;
  a.t = *t;
  a.N = M;
  a.C = C;
  a.F = F;
  int32_t *pf = nullptr, *bbo = nullptr;
  if ((rc = astra_market_portfolios(market, &pf))) return rc;
  if ((rc = astra_market_bbo_cache(market, &bbo))) return rc;
  a.portfolios = pf;
  a.bbo_cache = bbo;
  hipStream_t s = as_stream(stream);
  if ((rc = launch_pre(a, s))) return rc;
  if (t->check) {  // one wait, then stop like the reference's checks (:264-271)
    int32_t bits = 0;
    ASTRA_HIP_CHECK(rt_memcpy(&bits, t->errors, sizeof(bits), s), "error flags copy");
    ASTRA_HIP_CHECK(rt_sync(s), "error flags wait");
    if (bits) return fail(ASTRA_ERR_INVALID_ARGUMENT, std::string("high_low_trading.cc ") + check_text(bits));
  }
  const int64_t N = M;
  if (t->fill_rows)
    rc = astra_market_add_two_sided_quotes_rows(market, t->columns, t->columns + N,
                                                t->columns + 2 * N, t->columns + 3 * N,
                                                t->columns + 4 * N, t->fill_rows, t->fill_counts,
                                                stream);
  else
    rc = astra_market_add_two_sided_quotes(
        market, t->columns, t->columns + N, t->columns + 2 * N, t->columns + 3 * N,
        t->columns + 4 * N, t->fill_prices, t->fill_sizes, t->fill_customer_ids,
        t->fill_quoter_ids, t->fill_is_sell_quote, t->fill_quote_sizes, t->fill_tid,
        t->fill_quote_tid, t->fill_counts, stream);
  if (rc) return rc;
  return launch_post(a, s);
}

int astra_high_low_observation(const astra_hl_observation *o, void *stream) {
  ASTRA_ABI_CHECK(o != nullptr, ==, true);
  ASTRA_ABI_CHECK(o->num_envs, >=, 0);
  ASTRA_ABI_CHECK(o->players, >=, 1);
  ASTRA_ABI_CHECK(o->player, >=, 0);
  ASTRA_ABI_CHECK(o->player, <, o->players);
  ASTRA_ABI_CHECK(o->current_round, >=, 0);
  ASTRA_ABI_CHECK(o->current_round, <, o->steps_per_player);
  const int64_t total = (int64_t)o->num_envs * (6 + 1 + 6 * (int64_t)o->players + 5);
  if (total == 0) return ASTRA_OK;
  const void *need[] = {o->values, o->player_permutation, o->contract_values,
                        o->contract_high_settle, o->target_positions,
                        o->player_contract_over_time, o->best_bid_prices, o->best_ask_prices,
                        o->best_bid_sizes, o->best_ask_sizes, o->last_prices};
  for (const void *p : need)
    if (p == nullptr)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_high_low_observation: null pointer");
#ifdef ASTRA_HOST_EMULATION
  (void)stream;
  for (int64_t i = 0; i < total; ++i) observation_element(*o, i);
  return ASTRA_OK;
#else
  hipLaunchKernelGGL(observation_kernel, dim3(grid_for(total)), dim3(kBlock), 0,
                     as_stream(stream), *o, total);
  ASTRA_HIP_CHECK(rt_last_error(), "observation_kernel launch");
  return ASTRA_OK;
#endif
}

}  // extern "C"

/*
 * astra_high_low.h -- C ABI of the high-low trading game's per-move kernels on
 * MI355X (gfx950), around the VecMarket engine of astra_market.h.
 *
 * Replaces the hot path of nlyu1/astra-cuda
 * src/games/high_low_trading/high_low_trading.cc: the trading move
 * HighLowTradingState::ApplyPlayerTrading (:247-329) and
 * HighLowTradingState::FillObservationTensor (:510-602). The reference runs each
 * trading move as about forty libtorch kernels plus eight .item() host syncs for
 * its input checks and a host-to-device copy of the customer ids; here a move is
 * one launch of the matching kernel with the game's checks, portfolio snapshot,
 * BBO, last price, telemetry and rewards fused around each env's matching (plus,
 * with check = 1, a check launch and one host sync before it), and an
 * observation is one launch.
 *
 * All pointers are device pointers to int32 (uint8 for the bool settle flags,
 * float for observations), row-major and contiguous; the caller owns them.
 */
#ifndef ASTRA_HIGH_LOW_H
#define ASTRA_HIGH_LOW_H

#include <stddef.h>
#include <stdint.h>

#include "astra_market.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bits of *errors after a trading move whose input failed the reference's range
 * checks (high_low_trading.cc:264-271), one per check in that order. */
#define ASTRA_HL_ERR_BID_PRICE_LOW (1 << 0)  /* bid_px > 0 */
#define ASTRA_HL_ERR_ASK_PRICE_LOW (1 << 1)  /* ask_px > 0 */
#define ASTRA_HL_ERR_BID_PRICE_HIGH (1 << 2) /* bid_px <= max_contract_value */
#define ASTRA_HL_ERR_ASK_PRICE_HIGH (1 << 3) /* ask_px <= max_contract_value */
#define ASTRA_HL_ERR_BID_SIZE_LOW (1 << 4)   /* bid_sz >= 0 */
#define ASTRA_HL_ERR_ASK_SIZE_LOW (1 << 5)   /* ask_sz >= 0 */
#define ASTRA_HL_ERR_BID_SIZE_HIGH (1 << 6)  /* bid_sz <= max_contracts_per_trade */
#define ASTRA_HL_ERR_ASK_SIZE_HIGH (1 << 7)  /* ask_sz <= max_contracts_per_trade */

/* One trading move of every env (the state tensors of high_low_trading.h:85-115). */
typedef struct astra_hl_trade {
  const int32_t *move;            /* [N,4]: bid_px, ask_px, bid_sz, ask_sz (:260-263) */
  int32_t *player_last_positions; /* [N,P,2] */
  const int32_t *target_positions;/* [N,P] */
  const int32_t *contract_values; /* [N,3] */
  int32_t *player_contract_over_time; /* the reference's [N,P,T,6] tensor stored env-minor,
                                         as [T,P,6,N]: word (n,p,t,f) at ((t*P+p)*6+f)*N+n,
                                         so that consecutive envs' words are adjacent */
  int32_t *market_contract_over_time; /* the reference's [N,P*T,3] stored env-minor, as
                                         [P*T,3,N]: word (n,k,f) at (k*3+f)*N+n */
  int32_t *immediate_rewards;     /* [N,P] */
  int32_t *rewards_since_last_action; /* [N,P] */
  /* FillBatch (market.h:64-92) and BBOBatch (market.h:95-119) of the env's market */
  int32_t *fill_prices, *fill_sizes, *fill_customer_ids, *fill_quoter_ids;
  uint8_t *fill_is_sell_quote;
  int32_t *fill_quote_sizes, *fill_tid, *fill_quote_tid, *fill_counts;
  int32_t *best_bid_prices, *best_bid_sizes, *best_ask_prices, *best_ask_sizes, *last_prices;
  int32_t *fill_rows;             /* non-NULL: the fills go to this [N,F,8] row array
                                     (astra_market_add_two_sided_quotes_rows) and the
                                     eight field pointers above are not used */
  int32_t *errors;                /* [1]: ASTRA_HL_ERR_* bits are OR-ed in; the caller zeroes it */
  int32_t *errors_host;           /* NULL, or one int32 of pinned host memory: with check = 1
                                     the error word is copied there right after the checks and
                                     the host waits for that copy only, so the move kernel,
                                     already queued, runs while the call returns */
  int32_t players, steps_per_player, max_contracts_per_trade, max_contract_value;
  int32_t player;                 /* the acting player (CurrentPlayer) */
  int32_t trade_move_number;      /* MoveNumber() - MaxChanceNodesInHistory() */
  int32_t check;                  /* 1: return the reference's error, with no state
                                     changed, if any check failed (one host wait; the move
                                     kernel then leaves every env as it is); 0: no wait,
                                     the errors stay in *errors */
} astra_hl_trade;

/* HighLowTradingState::ApplyPlayerTrading (high_low_trading.cc:247-329) for all N
 * envs of `market` (N = its market count; C >= players customers). */
int astra_high_low_trade(astra_market *market, const astra_hl_trade *t, void *stream);

/* No counterpart in the reference: astra_high_low_trade for callers that cannot
 * allocate device memory (serving loops, harnesses that forbid hipMalloc). The
 * checks' error word is a word of the library's own per-device scratch (one
 * static device array of 64 int32 per GPU) instead of t->errors, which is
 * ignored and may be NULL: each market gets a word of its own on its first such
 * move, kept until the market is destroyed, so at most 64 live markets per GPU
 * use this entry point (the 65th gets an error). Requires check = 1 (the word is
 * cleared by every call, so unchecked moves could not report later) and
 * errors_host (one int32 of pinned host memory). Results and errors are those of
 * astra_high_low_trade. Allocates nothing: the first call on a device sets up
 * the scratch's device address and one event per word. Moves of different
 * markets never share a word or an event; moves of one market must be ordered
 * (one stream, or synchronised), as every call on a market must be. */
int astra_high_low_trade_scratch(astra_market *market, const astra_hl_trade *t, void *stream);

/* FillObservationTensor(player, values) (high_low_trading.cc:510-602). */
typedef struct astra_hl_observation {
  float *values;                  /* [N, 6 + 1 + 6P + 5] */
  const int32_t *player_permutation; /* [N,P] */
  const int32_t *contract_values; /* [N,3] */
  const uint8_t *contract_high_settle; /* [N] */
  const int32_t *target_positions;/* [N,P] */
  const int32_t *player_contract_over_time; /* [T,P,6,N], as astra_hl_trade keeps it */
  const int32_t *best_bid_prices, *best_ask_prices, *best_bid_sizes, *best_ask_sizes, *last_prices;
  int32_t num_envs, players, steps_per_player, player, current_round;
  float player_sin, player_cos;   /* sin, cos of 2*pi*player/P, computed in double (:532-534) */
  float round_fraction;           /* current_round / steps_per_player in float32 (:556-557) */
} astra_hl_observation;

int astra_high_low_observation(const astra_hl_observation *o, void *stream);

/* FillRewards (high_low_trading.cc:331-336) with player < 0: dst[i] = (float)src[i] for
 * all num_envs * players words; FillRewardsSinceLastAction (:338-343) with
 * 0 <= player < players: dst[n] = (float)src[n * players + player]. src is the
 * [N,P] int32 reward tensor, dst a contiguous float32 buffer. */
int astra_high_low_rewards(const int32_t *src, int64_t num_envs, int32_t players, int32_t player,
                           float *dst, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* ASTRA_HIGH_LOW_H */

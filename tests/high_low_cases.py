"""Shared high-low game scenarios for the oracle, emulated and GPU tests.

HAND_GAME is derived by hand from src/games/high_low_trading/high_low_trading.cc
and src/order_matching/market.cu (one env, four players, two steps each,
max_contract_value 30; the market shape the game derives, :57-69: L=31, O=16,
F=10, C=4). The expected values below were worked out on paper, not by running
any implementation:

  setup: candidate values (10, 20), settle high -> value 20; permutation
  (0, 1, 2, 3): players 0, 1 value cheaters, 2 the high-low cheater, 3 a
  customer with target +2.
  move 0 (p0) bid 12x2, ask 18x1: rests. move 1 (p1) bid 18x3 lifts p0's ask at
  18 (ask rests: earlier TID). move 2 (p2) sizes 0: nothing inserted, cheap
  signalling on the bid (price 10 != 1) costs 30, the ask at 30 == V is free.
  move 3 (p3) bid 26x2, ask 24x1: self-trade at 26 (bid rests), then the bid's
  remaining 1 lifts p1's ask at 25; self-trade penalty (1+1)*(26-24+1)*30 = 180.
  moves 4-7: bid 1x1 / ask 30x1, no trades; move 7 settles contracts at 20.
"""
import numpy as np

HAND_GAME = {
    "params": dict(players=4, steps_per_player=2, max_contracts_per_trade=5, customer_max_size=5,
                   max_contract_value=30, num_markets=1),
    "chance": [np.array([[10, 20]], np.int32), np.array([1], np.int32),
               np.array([[0, 1, 2, 3]], np.int32), np.array([[2]], np.int32)],
    "moves": [[12, 18, 2, 1], [18, 25, 3, 1], [10, 30, 0, 0], [26, 24, 2, 1],
              [1, 30, 1, 1], [1, 30, 1, 1], [1, 30, 1, 1], [1, 30, 1, 1]],
    # after each trading move: immediate rewards, rewards since last action, portfolios
    # (contracts, cash) per player, and the market row (best bid, best ask, last price)
    "immediate": [[0, 0, 0, 0], [18, -18, 0, 0], [0, 0, -30, 0], [0, 25, 0, -175],
                  [0, 0, 0, 0], [0, 0, 0, 0], [0, 0, 0, 0], [-20, 0, 0, 20]],
    "since_last": [[0, 0, 0, 0], [18, -18, 0, 0], [18, -18, -30, 0], [18, 7, -30, -175],
                   [0, 7, -30, -175], [0, 0, -30, -175], [0, 0, 0, -175], [-20, 0, 0, 20]],
    "portfolios_after": {1: [[-1, 18], [1, -18], [0, 0], [0, 0]],
                         3: [[-1, 18], [0, 7], [0, 0], [1, -25]],
                         7: [[-1, 18], [0, 7], [0, 0], [1, -25]]},
    "market_rows": [[12, 18, 0], [18, 25, 18], [18, 25, 18], [18, -1, 25],
                    [18, 30, 25], [18, 30, 25], [18, 30, 25], [18, 30, 25]],
    "returns": [-2, 7, 0, -35],
    # observation of player 2 after move 5 (move number 10, round 1)
    "obs_after": 5,
    "obs_player": 2,
    "obs": [0, 1, 0, float(np.float32(np.sin(np.pi))), -1, 1, 0.5,
            1, 30, 1, 1, -1, 18, 1, 30, 1, 1, 0, 7, 10, 30, 0, 0, 0, 0, 26, 24, 2, 1, 1, -25,
            18, 30, 2, 1, 25],
    # The other round selections of :559-584. Each move writes its quote into the
    # acting player's row of the current round and every player's contracts and
    # cash after the move into all rows of that round (:290-291); rows of a round
    # not reached yet are zeros. Positions (contracts, cash): all (0, 0) after
    # move 0; after moves 1-2 p0 (-1, 18), p1 (1, -18); after moves 3-7 p0 (-1, 18),
    # p1 (0, 7), p2 (0, 0), p3 (1, -25). The last five words are the BBO and last
    # price after the move (bid px, ask px, bid sz, ask sz, last); sin and cos of
    # 2*pi*player/P are computed in double and stored as float32 (:532-534).
    "more_obs": [
        # round 0 (current_round == 0): player 1 after move 1 sees round 0 so far
        # (players 2 and 3 have not quoted yet); a value cheater with candidate 20
        (1, 1, [1, 0, 0, float(np.float32(np.sin(np.pi / 2))), float(np.float32(np.cos(np.pi / 2))),
                20, 0.0,
                12, 18, 2, 1, -1, 18, 18, 25, 3, 1, 1, -18, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                18, 25, 2, 1, 18]),
        # player 0 in round 1 (after move 5) sees all of round 0
        (5, 0, [1, 0, 0, 0.0, 1.0, 10, 0.5,
                12, 18, 2, 1, -1, 18, 18, 25, 3, 1, 0, 7, 10, 30, 0, 0, 0, 0, 26, 24, 2, 1, 1, -25,
                18, 30, 2, 1, 25]),
        # the last player (3) in round 1 (after move 6) sees round 1 so far: its own
        # quote not yet written, its position already; a customer with target 2
        (6, 3, [0, 0, 1, float(np.float32(np.sin(3 * np.pi / 2))),
                float(np.float32(np.cos(3 * np.pi / 2))), 2, 0.5,
                1, 30, 1, 1, -1, 18, 1, 30, 1, 1, 0, 7, 1, 30, 1, 1, 0, 0, 0, 0, 0, 0, 1, -25,
                18, 30, 2, 1, 25]),
    ],
}


def random_game(rng, N, P, T, S, cM, V):
    """Chance moves and trading moves like the reference's env.py (:42-56), plus
    prices and sizes over the full legal range (and some crossing quotes)."""
    cand = rng.integers(1, V + 1, (N, 2)).astype(np.int32)
    hl = rng.integers(0, 2, (N,)).astype(np.int32)
    perm = np.argsort(rng.random((N, P)), axis=1).astype(np.int32)
    cs = rng.integers(-cM, cM, (N, P - 3)).astype(np.int32)
    cs[cs >= 0] += 1
    moves = []
    for _ in range(T * P):
        mid = rng.integers(1, V + 1, (N,))
        bid = np.clip(mid + rng.integers(-4, 3, N), 1, V)
        ask = np.clip(mid + rng.integers(-2, 5, N), 1, V)
        moves.append(np.stack([bid, ask, rng.integers(0, S + 1, N), rng.integers(0, S + 1, N)],
                              1).astype(np.int32))
    return [cand, hl, perm, cs], moves


# Text of the hand game after move 3 (move number 8), worked out from
# high_low_trading.cc:398-466 and :620-804; the market's own book text follows the
# "Current Market" banner (pinned by the string_representation known-answer test).
HAND_TEXT_AFTER = 3
HAND_SETUP_TEXT = (
    "********** Game setup **********\n"
    "Contract values: 10, 20\n"
    "Contract high settle: High\n"
    "Player permutation: Player roles: P0=ValueCheater, P1=ValueCheater, P2=HighLowCheater, P3=Customer\n"
    "Player 0 target position: No requirement\n"
    "Player 1 target position: No requirement\n"
    "Player 2 target position: No requirement\n"
    "Player 3 target position: 2\n"
    "********************************\n\n")
HAND_PUBLIC_TEXT = (
    "********** Game Configuration **********\n"
    "Environment: 0 / 1\n"
    "Steps per player: 2\n"
    "Max contracts per trade: 5\n"
    "Customer max size: 5\n"
    "Max contract value: 30\n"
    "Number of players: 4\n"
    "****************************************\n\n"
    "********** Player Positions **********\n"
    "Player 0 position: [-1 contracts, 18 cash]\n"
    "Player 1 position: [0 contracts, 7 cash]\n"
    "Player 2 position: [0 contracts, 0 cash]\n"
    "Player 3 position: [1 contracts, -25 cash]\n"
    "**************************************\n\n"
    "********** Quotes & Market Movement **********\n"
    "Number of fills in the last round: 2\n"
    "Order fill: id=3 sold 1 contracts at px=26 on t=7. Quote: id=3 bid sz=2, submitted t=6\n"
    "Order fill: id=3 bought 1 contracts at px=25 on t=6. Quote: id=1 sale sz=1, submitted t=3\n"
    "Player 0 quote: 12 @ 18 [2 x 1]\n"
    "Player 1 quote: 18 @ 25 [3 x 1]\n"
    "Player 2 quote: 10 @ 30 [0 x 0]\n"
    "Player 3 quote: 26 @ 24 [2 x 1]\n"
    "\n--- Market Movement ---\n"
    "Time 0: Bid: 12 @ Ask: 18, Last: 0\n"
    "Time 1: Bid: 18 @ Ask: 25, Last: 18\n"
    "Time 2: Bid: 18 @ Ask: 25, Last: 18\n"
    "Time 3: Bid: 18 @ Ask: none, Last: 25\n"
    "***********************************\n\n"
    "********** Current Market **********\n")
HAND_PRIVATE_TEXT = {
    0: "My role: ValueCheater\nCandidate contract value: 10\n",
    2: "My role: HighLowCheater\nSettlement will be: High\n",
    3: "My role: Customer\nMy target position: 2\n",
}

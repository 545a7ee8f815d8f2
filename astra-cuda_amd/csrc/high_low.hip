// high_low.hip -- the high-low trading game's per-move kernels (MI355X, gfx950)
// behind the C ABI of include/astra_high_low.h.
//
// Semantics follow nlyu1/astra-cuda src/games/high_low_trading/high_low_trading.cc:
// the trading move HighLowTradingState::ApplyPlayerTrading (:247-329) and
// FillObservationTensor (:510-602). The reference spreads a move over about forty
// libtorch launches and eight .item() syncs; here the whole move is one launch
// of the VecMarket matching kernel with the game's work fused around each
// market's matching (game_move.h: checks, portfolio snapshot, BBO, last price,
// telemetry, rewards). With check = 1 a small kernel checks the move's ranges
// first, the move kernel leaves every env untouched when any check failed, and
// the host waits once, after the move, and returns the reference's error; with
// check = 0 nothing waits and the failed checks stay in *errors.
//
// The kernel bodies are __host__ __device__ functions; the host-emulation build
// (-DASTRA_HOST_EMULATION) runs them as loops over host memory.
#include <cmath>
#include <mutex>
#include <string>

#include "astra_high_low.h"

#define ASTRA_SRC_NAME "high_low.hip"
#include "runtime.h"
#include "game_move.h"

using namespace astra_rt;

namespace {

constexpr int kBlock = 256;

// The observation and reward tensors are written once per call and read later by
// the caller, never by these kernels: non-temporal stores stream them past the
// caches, which keep the move's books (the observation of 262,144 envs, 44 MB:
// the game step about 3% faster). The observation's column loads, each word read
// once per call, are non-temporal too.
typedef float f32x4 __attribute__((ext_vector_type(4)));

static_assert(ASTRA_HL_ERR_BID_PRICE_LOW == 1 && ASTRA_HL_ERR_ASK_PRICE_LOW == 2 &&
                  ASTRA_HL_ERR_BID_PRICE_HIGH == 4 && ASTRA_HL_ERR_ASK_PRICE_HIGH == 8 &&
                  ASTRA_HL_ERR_BID_SIZE_LOW == 16 && ASTRA_HL_ERR_ASK_SIZE_LOW == 32 &&
                  ASTRA_HL_ERR_BID_SIZE_HIGH == 64 && ASTRA_HL_ERR_ASK_SIZE_HIGH == 128,
              "game_quote's check bits");

// The range checks of env n's move (high_low_trading.cc:264-271).
ASTRA_HD void trade_check(const GameMove &g, int64_t n) {
  const int32_t bad = game_quote(g, n).bad;
  if (bad) {
#if defined(__HIP_DEVICE_COMPILE__)
    atomicOr(g.errors, bad);
#else
    *g.errors |= bad;
#endif
  }
}

// One element of the [N, 6 + 1 + 6P + 5] observation (:510-602).
ASTRA_HD void observation_element(const astra_hl_observation &o, int64_t i) {
  const int32_t P = o.players, player = o.player, cr = o.current_round;
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
    v = (float)o.player_contract_over_time[(((int64_t)r * P + p) * 6 + f) * o.num_envs + n];
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

// The checks of every env OR-ed into g.errors. With `errors_host` (pinned host
// memory, zeroed by the host before the launch), a workgroup with a failed
// check also stores its bits there, so that the host learns whether any check
// failed without a copy on the stream; it reads the exact bits from g.errors
// only then.
__global__ __launch_bounds__(kBlock) void trade_check_kernel(GameMove g, int64_t N, int32_t *errors_host) {
  __shared__ int32_t acc;
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (threadIdx.x == 0) acc = 0;
  __syncthreads();
  const int32_t bad = n < N ? game_quote(g, n).bad : 0;
  if (bad) atomicOr(&acc, bad);
  __syncthreads();
  if (threadIdx.x == 0 && acc) {
    atomicOr(g.errors, acc);
    if (errors_host) __hip_atomic_store(errors_host, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

__global__ __launch_bounds__(kBlock) void observation_kernel(astra_hl_observation o, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < total) observation_element(o, i);
}

// Column j's source (:510-602): kind 0 = one-hot of the permutation entry
// (j 0-2), 1 = a constant (j 3, 4, 6), 2 = the private information (j 5),
// 3 = src[n * stride] (the rounds of player_contract_over_time, then the BBO and
// last-price arrays). Kinds 0-2 read the permutation entry as their word.
struct ObsColumn {
  const int32_t *src;
  int64_t stride;
  int32_t kind;
  float constant;
};

ASTRA_HD ObsColumn obs_column(const astra_hl_observation &o, int32_t j) {
  const int32_t P = o.players, player = o.player, cr = o.current_round;
  ObsColumn c{o.player_permutation + player, P, 0, 0.0f};
  if (j <= 2) {
    c.kind = 0;
  } else if (j == 3 || j == 4 || j == 6) {
    c.kind = 1;
    c.constant = j == 3 ? o.player_sin : j == 4 ? o.player_cos : o.round_fraction;
  } else if (j == 5) {
    c.kind = 2;
  } else if (j < 7 + 6 * P) {  // the round of player p shown to `player` (:559-584)
    const int32_t q = j - 7, p = q / 6, f = q - 6 * (q / 6);
    int32_t r;
    if (cr == 0 || player == P - 1) r = cr;
    else if (player == 0) r = cr - 1;
    else r = p < player ? cr : cr - 1;
    c.src = o.player_contract_over_time + (((int64_t)r * P + p) * 6 + f) * o.num_envs;
    c.stride = 1;
    c.kind = 3;
  } else {  // BBO and last price (:589-599)
    const int32_t k = j - (7 + 6 * P);
    c.src = k == 0   ? o.best_bid_prices
            : k == 1 ? o.best_ask_prices
            : k == 2 ? o.best_bid_sizes
            : k == 3 ? o.best_ask_sizes
                     : o.last_prices;
    c.stride = 1;
    c.kind = 3;
  }
  return c;
}

// Column j's value for one env from its loaded words (observation_element's
// cases, in the same order).
ASTRA_HD float obs_value(const ObsColumn &c, int32_t j, int32_t perm, int32_t word, int32_t cv0,
                         int32_t cv1, uint8_t settle, int32_t target) {
  if (c.kind == 0)
    return (j == 0 ? (perm == 0 || perm == 1) : j == 1 ? perm == 2 : perm > 2) ? 1.0f : 0.0f;
  if (c.kind == 1) return c.constant;
  if (c.kind == 2) {
    if (perm == 0) return (float)cv0;
    if (perm == 1) return (float)cv1;
    if (perm == 2) return settle ? 1.0f : 0.0f;
    if (perm > 2) return (float)target;
    return 0.0f;
  }
  return (float)word;
}

// Column j of env n (the host build's loop; the kernel below loads the same words).
ASTRA_HD void observation_column(const astra_hl_observation &o, int64_t n, int32_t j) {
  const ObsColumn c = obs_column(o, j);
  const int32_t P = o.players, D = 12 + 6 * P;
  o.values[n * D + j] =
      obs_value(c, j, o.player_permutation[n * P + o.player], c.src[n * c.stride],
                o.contract_values[n * 3], o.contract_values[n * 3 + 1],
                o.contract_high_settle[n], o.target_positions[n * P + o.player]);
}

// The same observation with one lane per env, for rows of at most 64 columns
// (P <= 8). A column's source is fixed for the call, and consecutive envs' words
// are adjacent in every source (the env-minor player_contract_over_time, the [N]
// BBO arrays), so a wavefront loads each column of its 64 envs with one
// coalesced load, all columns before any wait (the per-element kernel above
// branches on the column and waits once per branch); it transposes the values in
// LDS. Its 64 rows are one contiguous block of 64 * D floats in `values`, which
// the wavefront writes as a flat array: 16 bytes per lane and store (`vec`: the
// block is 16-byte aligned, since n0 * D * 4 is a multiple of 256 and `values`
// is 16-byte aligned), else 4 bytes per lane; every store covers 1 KB (or
// 256 B) of consecutive addresses.
constexpr int kObsTileWaves = 2;     // wavefronts per block

template <int PP>
__global__ __launch_bounds__(kObsTileWaves * 64) void observation_tile_kernel(astra_hl_observation o,
                                                                             int64_t N, int32_t vec) {
  constexpr int32_t D = 12 + 6 * PP;  // row length; the player count is a template argument
  constexpr int32_t pitch = D + 1;    // odd (D is even): lanes' rows fall in different banks
  extern __shared__ float obs_tile[];  // per wavefront: 64 rows of `pitch` floats
  const int lane = (int)(threadIdx.x % 64), w = (int)(threadIdx.x / 64);
  const int64_t n0 = ((int64_t)blockIdx.x * kObsTileWaves + w) * 64;
  const int32_t player = o.player;
  const int64_t n = n0 + lane < N ? n0 + lane : N - 1;  // clamped: no branch around a load
  // the env's own words (role, private information), then one coalesced load per
  // column of the rounds and the BBO, all issued before any wait
  const int32_t perm = o.player_permutation[n * PP + player];
  const int32_t cv0 = o.contract_values[n * 3], cv1 = o.contract_values[n * 3 + 1];
  const uint8_t settle = o.contract_high_settle[n];
  const int32_t target = o.target_positions[n * PP + player];
  int32_t word[D];
#pragma unroll
  for (int32_t j = 7; j < D; ++j) {
    const ObsColumn c = obs_column(o, j);
    word[j] = __builtin_nontemporal_load(c.src + n * c.stride);  // read once per call
  }
  float *tile = obs_tile + w * 64 * pitch;
#pragma unroll
  for (int32_t j = 0; j < D; ++j)
    tile[lane * pitch + j] =
        obs_value(obs_column(o, j), j, perm, j < 7 ? perm : word[j], cv0, cv1, settle, target);
  __syncthreads();
  const int64_t rows = N - n0 < 64 ? N - n0 : 64;
  if (rows <= 0) return;
  const int32_t total = (int32_t)rows * D;  // floats of this wavefront's rows
  float *dst = o.values + n0 * D;
  // flat index f of the block is row f / D, column f % D of the tile
  if (vec && rows == 64) {
    for (int32_t f = lane * 4; f < total; f += 256) {
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int32_t e = (f + q) / D, jj = (f + q) - e * D;
        v[q] = tile[e * pitch + jj];
      }
      __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4 *>(dst + f));
    }
  } else {
    for (int32_t f = lane; f < total; f += 64) {
      const int32_t e = f / D, jj = f - e * D;
      __builtin_nontemporal_store(tile[e * pitch + jj], dst + f);
    }
  }
}

template <int PP>
void launch_observation_tile(const astra_hl_observation &o, hipStream_t s) {
  const int64_t per_block = 64 * kObsTileWaves;
  const unsigned blocks = (unsigned)(((int64_t)o.num_envs + per_block - 1) / per_block);
  const size_t lds = (size_t)per_block * (13 + 6 * PP) * sizeof(float);
  const int32_t vec = reinterpret_cast<uintptr_t>(o.values) % 16 == 0 ? 1 : 0;
  hipLaunchKernelGGL(observation_tile_kernel<PP>, dim3(blocks), dim3(per_block), lds, s, o,
                     (int64_t)o.num_envs, vec);
}

// The rewards as float32: column `col` of the [n, stride] int32 array (col >= 0),
// or all n words, four per lane with 16-byte accesses when `vec` (both pointers
// 16-byte aligned). A plain int32 -> float32 conversion, as libtorch's copy_.
__global__ __launch_bounds__(kBlock) void rewards_kernel(const int32_t *src, float *dst, int64_t n,
                                                         int32_t stride, int32_t col, int32_t vec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= 0) {
    if (i < n) __builtin_nontemporal_store((float)src[i * stride + col], dst + i);
  } else if (vec) {
    const int64_t k = i * 4;
    if (k + 4 <= n) {
      const int4 v = *reinterpret_cast<const int4 *>(src + k);
      __builtin_nontemporal_store(f32x4{(float)v.x, (float)v.y, (float)v.z, (float)v.w},
                                  reinterpret_cast<f32x4 *>(dst + k));
    } else {
      for (int64_t q = k; q < n; ++q) __builtin_nontemporal_store((float)src[q], dst + q);
    }
  } else if (i < n) {
    __builtin_nontemporal_store((float)src[i], dst + i);
  }
}

inline unsigned grid_for(int64_t n) { return (unsigned)((n + kBlock - 1) / kBlock); }

// errors_host: see trade_check_kernel (the host zeroes it here, before the launch;
// no earlier launch that may store to it is still running, since the host waited
// for the last check).
int launch_check(const GameMove &g, int64_t N, int32_t *errors_host, hipStream_t s) {
  if (errors_host) *errors_host = 0;
#ifdef ASTRA_HOST_EMULATION
  (void)s;
  for (int64_t n = 0; n < N; ++n) trade_check(g, n);
  if (errors_host) *errors_host = *g.errors;
  return ASTRA_OK;
#else
  if (N > 0)
    hipLaunchKernelGGL(trade_check_kernel, dim3(grid_for(N)), dim3(kBlock), 0, s, g, N, errors_host);
  ASTRA_HIP_CHECK(rt_last_error(), "trade_check_kernel launch");
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

// The error words of astra_high_low_trade_scratch: the library's own device
// memory, so that its callers need not allocate any. Each GPU holds its own copy
// at its own address (kept per device in g_scratch after hipGetSymbolAddress);
// in host code the array's name is not a device address and is never used as
// one. Each market that makes such a move gets a word of its own for the failed
// checks' bits of its moves (and an event of its own for their completion), so
// moves of different markets never share one; at most kScratchWords live
// markets per GPU, a destroyed market's word goes back to the pool.
constexpr int kScratchWords = 64;
#ifdef ASTRA_HOST_EMULATION
static int32_t scratch[kScratchWords];  // the host build keeps its "device" memory on the host
#else
static __device__ __align__(256) int32_t scratch[kScratchWords];
#endif

namespace {

constexpr int kMaxScratchDevices = 64;
struct ScratchDevice {
  int32_t *ptr = nullptr;               // device address of `scratch` on this device
  hipEvent_t ev[kScratchWords] = {};    // the checks' completion event of each word
  uint64_t used = 0;                    // words held by live markets
};
ScratchDevice g_scratch[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Set-up, once per device with that device current (the device's first
// allocation-free move): the address of its copy of `scratch` and one event per
// word, so that the calls themselves allocate nothing. Then the market's word,
// assigned on its first such move.
int scratch_word(astra_market *market, int dev, ScratchDevice **out, int *word) {
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_high_low_trade_scratch: device id out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchDevice &d = g_scratch[dev];
  if (!d.ptr) {
#ifdef ASTRA_HOST_EMULATION
    d.ptr = scratch;  // the host build's "device" memory is host memory
#else
    DeviceGuard g(dev);
    if (!g.ok) return fail(ASTRA_ERR_HIP, "hipSetDevice failed");
    int32_t *p = nullptr;
    ASTRA_HIP_CHECK(hipGetSymbolAddress(reinterpret_cast<void **>(&p), HIP_SYMBOL(scratch)),
                    "hipGetSymbolAddress(scratch)");
    for (int i = 0; i < kScratchWords; ++i)
      if (!d.ev[i])
        ASTRA_HIP_CHECK(hipEventCreateWithFlags(&d.ev[i], hipEventDisableTiming),
                        "hipEventCreateWithFlags");
    d.ptr = p;
#endif
  }
  int w = astra_game_scratch_word(market);
  if (w < 0) {
    if (d.used == ~0ull)
      return fail(ASTRA_ERR_INVALID_ARGUMENT,
                  "astra_high_low_trade_scratch: all " + std::to_string(kScratchWords) +
                      " scratch words of device " + std::to_string(dev) +
                      " are held by live markets");
    w = __builtin_ctzll(~d.used);
    d.used |= 1ull << w;
    astra_game_set_scratch_word(market, w);
  }
  *out = &d;
  *word = w;
  return ASTRA_OK;
}

// ApplyPlayerTrading for all envs of `market` (astra_high_low_trade), with the
// checks' error word at `errors` and, when set, `ev` as the checks' event.
int trade_impl(astra_market *market, const astra_hl_trade *t, int32_t *errors, hipEvent_t ev,
               void *stream) {
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
  const void *need[] = {t->move, t->player_last_positions, t->target_positions,
                        t->contract_values, t->player_contract_over_time,
                        t->market_contract_over_time, t->immediate_rewards,
                        t->rewards_since_last_action, t->fill_counts, t->best_bid_prices,
                        t->best_bid_sizes, t->best_ask_prices, t->best_ask_sizes,
                        t->last_prices, errors};
  for (const void *p : need)
    if (M > 0 && p == nullptr)
      return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_high_low_trade: null pointer in astra_hl_trade");
  int32_t *const fields[8] = {t->fill_prices, t->fill_sizes, t->fill_customer_ids, t->fill_quoter_ids,
                              reinterpret_cast<int32_t *>(t->fill_is_sell_quote), t->fill_quote_sizes,
                              t->fill_tid, t->fill_quote_tid};
  if (!t->fill_rows)
    for (const int32_t *p : fields)
      if (M > 0 && p == nullptr)
        return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_high_low_trade: null fill pointer");
  GameMove g;
  g.move = t->move;
  g.last_pos = t->player_last_positions;
  g.target = t->target_positions;
  g.contract_values = t->contract_values;
  g.pcot = t->player_contract_over_time;
  g.mcot = t->market_contract_over_time;
  g.imm = t->immediate_rewards;
  g.rsla = t->rewards_since_last_action;
  g.bbo_out[0] = t->best_bid_prices;
  g.bbo_out[1] = t->best_bid_sizes;
  g.bbo_out[2] = t->best_ask_prices;
  g.bbo_out[3] = t->best_ask_sizes;
  g.last_prices = t->last_prices;
  g.errors = errors;
  g.P = t->players;
  g.T = t->steps_per_player;
  g.S = t->max_contracts_per_trade;
  g.V = t->max_contract_value;
  g.player = t->player;
  g.tmn = t->trade_move_number;
  hipStream_t s = as_stream(stream);
  DeviceGuard dg(astra_game_device(market));
  // With checks (the reference's behaviour, :264-271): a check launch, the error
  // word to the host, then the move, which leaves every env as it is, and the
  // TID counter too, when any check failed; so the call has changed nothing when
  // it returns the error. The host waits for the checks (with errors_host, only
  // for them: the move runs meanwhile).
  g.abort_on_error = t->check ? 1 : 0;
  int32_t bits = 0;
  StreamMark checked;
  checked.ev = ev;
  if (t->check) {
    // (with errors_host a failed check's workgroup marks it there itself)
    if ((rc = launch_check(g, M, t->errors_host, s))) return rc;
    if (t->errors_host) ASTRA_HIP_CHECK(checked.record(s), "error flags event");
  }
  // the move itself: one launch of the matching kernel with the game's work fused
  if ((rc = astra_game_move(market, g, fields, t->fill_rows, t->fill_counts, s))) return rc;
  if (!t->check) return ASTRA_OK;
  if (t->errors_host) {
    ASTRA_HIP_CHECK(checked.wait(), "error flags wait");
    bits = *t->errors_host;
    if (bits) {  // a check failed: all of them, from the device word (the checks are done)
      ASTRA_HIP_CHECK(rt_memcpy(&bits, errors, sizeof(bits), s), "error flags copy");
      ASTRA_HIP_CHECK(rt_sync(s), "error flags wait");
    }
  } else {
    ASTRA_HIP_CHECK(rt_memcpy(&bits, errors, sizeof(bits), s), "error flags copy");
    ASTRA_HIP_CHECK(rt_sync(s), "error flags wait");
  }
  if (bits) {
    return fail(ASTRA_ERR_INVALID_ARGUMENT, std::string("high_low_trading.cc ") + check_text(bits));
  }
  return ASTRA_OK;
}

}  // namespace

extern "C" {

int astra_high_low_trade(astra_market *market, const astra_hl_trade *t, void *stream) {
  ASTRA_ABI_CHECK(t != nullptr, ==, true);
  return trade_impl(market, t, t->errors, nullptr, stream);
}

int astra_high_low_trade_scratch(astra_market *market, const astra_hl_trade *t, void *stream) {
  ASTRA_ABI_CHECK(market != nullptr, ==, true);
  ASTRA_ABI_CHECK(t != nullptr, ==, true);
  if (t->check != 1)
    return fail(ASTRA_ERR_INVALID_ARGUMENT,
                "astra_high_low_trade_scratch: check must be 1 (the error word is the library's "
                "scratch, cleared by every call, so unchecked moves could not report later)");
  if (!t->errors_host)
    return fail(ASTRA_ERR_INVALID_ARGUMENT,
                "astra_high_low_trade_scratch: errors_host (one int32 of pinned host memory) is "
                "required");
  ScratchDevice *d = nullptr;
  int w = 0;
  int rc = scratch_word(market, astra_game_device(market), &d, &w);
  if (rc) return rc;
  // the market's word starts at zero: a fill kernel (its last move left its bits there)
  if ((rc = astra_fill_i32(d->ptr + w, 1, 0, stream))) return rc;
  return trade_impl(market, t, d->ptr + w, d->ev[w], stream);
}

}  // extern "C"

void astra_game_release_scratch_word(int device, int word) {
  if (device < 0 || device >= kMaxScratchDevices || word < 0 || word >= kScratchWords) return;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  g_scratch[device].used &= ~(1ull << word);
}

extern "C" {

int astra_high_low_rewards(const int32_t *src, int64_t num_envs, int32_t players, int32_t player,
                           float *dst, void *stream) {
  ASTRA_ABI_CHECK(num_envs, >=, 0);
  ASTRA_ABI_CHECK(players, >=, 1);
  ASTRA_ABI_CHECK(player, <, players);
  const int64_t n = player < 0 ? num_envs * players : num_envs;
  if (n == 0) return ASTRA_OK;
  if (src == nullptr || dst == nullptr)
    return fail(ASTRA_ERR_INVALID_ARGUMENT, "astra_high_low_rewards: null pointer");
  const int32_t col = player < 0 ? -1 : player;
#ifdef ASTRA_HOST_EMULATION
  (void)stream;
  for (int64_t i = 0; i < n; ++i) dst[i] = (float)(col < 0 ? src[i] : src[i * players + col]);
  return ASTRA_OK;
#else
  const int32_t vec = col < 0 && ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0);
  const int64_t lanes = vec ? (n + 3) / 4 : n;
  hipLaunchKernelGGL(rewards_kernel, dim3(grid_for(lanes)), dim3(kBlock), 0, as_stream(stream), src,
                     dst, n, players, col, vec);
  ASTRA_HIP_CHECK(rt_last_error(), "rewards_kernel launch");
  return ASTRA_OK;
#endif
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
  const bool rows = 12 + 6 * (int64_t)o->players <= 64;  // one lane per column
#ifdef ASTRA_HOST_EMULATION
  (void)stream;
  if (rows) {
    for (int64_t n = 0; n < o->num_envs; ++n)
      for (int32_t j = 0; j < 12 + 6 * o->players; ++j) observation_column(*o, n, j);
  } else {
    for (int64_t i = 0; i < total; ++i) observation_element(*o, i);
  }
  return ASTRA_OK;
#else
  if (rows) {
    switch (o->players) {
      case 1: launch_observation_tile<1>(*o, as_stream(stream)); break;
      case 2: launch_observation_tile<2>(*o, as_stream(stream)); break;
      case 3: launch_observation_tile<3>(*o, as_stream(stream)); break;
      case 4: launch_observation_tile<4>(*o, as_stream(stream)); break;
      case 5: launch_observation_tile<5>(*o, as_stream(stream)); break;
      case 6: launch_observation_tile<6>(*o, as_stream(stream)); break;
      case 7: launch_observation_tile<7>(*o, as_stream(stream)); break;
      default: launch_observation_tile<8>(*o, as_stream(stream)); break;
    }
  } else {
    hipLaunchKernelGGL(observation_kernel, dim3(grid_for(total)), dim3(kBlock), 0,
                       as_stream(stream), *o, total);
  }
  ASTRA_HIP_CHECK(rt_last_error(), "observation_kernel launch");
  return ASTRA_OK;
#endif
}

}  // extern "C"

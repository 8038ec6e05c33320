/* nesle_ppo.h -- the clipped-PPO loss head of libnesle_hip.so.
 *
 * Plain C over device pointers: float32 tensors, int64 actions, work enqueued
 * on the caller's HIP stream (nothing is allocated, nothing synchronises, no
 * memset: the call may be captured in a graph).  Status codes and
 * nesle_last_error() are those of nesle_hip.h.
 */
#ifndef NESLE_PPO_H
#define NESLE_PPO_H

#include <stdint.h>

#include "nesle_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define NESLE_PPO_MAX_ACTIONS 1024u
/* Largest minibatch nesle_ppo_head_static takes (its static scratch). */
#define NESLE_PPO_STATIC_MAX_BATCH 1048576u

/* Floats of scratch nesle_ppo_head needs for a minibatch of `batch` rows. */
uint32_t nesle_ppo_head_scratch_floats(uint32_t batch);

/* The loss of one PPO minibatch and its gradient, replacing the loss lines
 * of the reference trainer (src/nesle/native_ppo.py:546-566: Categorical
 * log-probability and entropy of `logits`, ratio against `old_logprob`,
 * advantages normalised by their mean and unbiased standard deviation + 1e-8,
 * the clipped surrogate max(-A r, -A clamp(r, 1 - clip, 1 + clip)), the value
 * loss 0.5 (value - return)^2, all as means over the rows; loss =
 * surrogate - ent_coef * entropy + vf_coef * value loss).
 *
 *   logits [batch, num_actions], value [batch], actions [batch] (int64, in
 *   0..num_actions-1; another value makes that row's terms NaN),
 *   old_logprob, advantages, returns [batch]: inputs, contiguous.
 *   dlogits [batch, num_actions], dvalue [batch]: d loss / d input for a
 *   loss gradient of 1 (the autograd backward scales them).
 *   scratch: nesle_ppo_head_scratch_floats(batch) floats.
 *   loss, clipfrac: one float each (clipfrac = mean of |r - 1| > clip).
 *   accum: null, or two floats to which loss and clipfrac are added.
 *
 * Fails with NESLE_EINVAL for batch 0, num_actions outside
 * 1..NESLE_PPO_MAX_ACTIONS or a null pointer (other than accum). */
int nesle_ppo_head(const float* logits, const float* value, const int64_t* actions, const float* old_logprob,
                   const float* advantages, const float* returns, uint32_t batch, uint32_t num_actions,
                   double clip_coef, double ent_coef, double vf_coef, float* dlogits, float* dvalue,
                   float* scratch, float* loss, float* clipfrac, float* accum, void* stream);

/* nesle_ppo_head without the scratch argument: the same kernels on a
 * library-owned scratch array of static device storage (64 KiB per device,
 * held until the process ends), so the call allocates nothing.  No
 * counterpart in the reference: for callers that cannot allocate or be
 * handed a workspace, such as code under HIP graph capture or a serving
 * loop that forbids allocation.  The current device must be the one the
 * pointers and the stream belong to.  Every call on a device shares that
 * device's scratch: calls that overlap on one GPU (other streams, other
 * threads) race; calls in order on one stream do not.  Fails with
 * NESLE_EINVAL as nesle_ppo_head, and for batch > NESLE_PPO_STATIC_MAX_BATCH. */
int nesle_ppo_head_static(const float* logits, const float* value, const int64_t* actions, const float* old_logprob,
                          const float* advantages, const float* returns, uint32_t batch, uint32_t num_actions,
                          double clip_coef, double ent_coef, double vf_coef, float* dlogits, float* dvalue,
                          float* loss, float* clipfrac, float* accum, void* stream);

/* ---- the shaped Super Mario Bros. reward of the trainer ----------------------
 * The reference trainer's reward_mode="smart" (src/nesle/native_ppo.py:120-316,
 * TorchSmartMarioReward): progress, checkpoints, score, kills, coins, finish
 * zone, flag, stalling, button, death and time terms from the env-step's RAM,
 * pad masks and done flags, one thread per console, float32 rounded as
 * PyTorch rounds it (bit-identical to the reference's tensor arithmetic).
 * Device pointers, work on the caller's stream; nothing allocated, nothing
 * synchronised (capturable in a graph). */

/* 32-bit words of tracking state per console ([11][n], row-major). */
#define NESLE_SMB_SHAPED_STATE_WORDS 11u

/* The reward's constants (TorchSmartMarioReward's class attributes). */
typedef struct nesle_smb_shaped_params {
    float progress_scale, backtrack_scale, checkpoint_bonus, checkpoint_width, score_scale, coin_bonus, kill_bonus;
    float finish_zone_x, finish_zone_bonus, flag_zone_x, flag_bonus, death_penalty, time_penalty;
    float stall_penalty, max_stall_penalty, jump_penalty, neutral_jump_penalty, repeated_jump_penalty;
    float max_repeated_jump_penalty, left_penalty, bad_button_penalty;
    int32_t stall_window, repeated_jump_window;
} nesle_smb_shaped_params;

/* The reference's values (native_ppo.py:135-157). */
void nesle_smb_shaped_defaults(nesle_smb_shaped_params* params);

/* Start episodes: the tracking state of consoles with mask[e] != 0 (mask
 * null = all) from their RAM (ram: [n][2048] env-major).  Replaces
 * reset/reset_where (native_ppo.py:171-207). */
int nesle_smb_shaped_reset(const uint8_t* ram, const uint8_t* mask, uint32_t n, void* state, void* stream);

/* Reward of one env-step into reward[n] from the step's RAM (before any
 * reset), pad masks and done flags (uint8 [n] each); updates the state.
 * Replaces compute (native_ppo.py:209-278). */
int nesle_smb_shaped_reward(const uint8_t* ram, const uint8_t* pads, const uint8_t* dones, uint32_t n,
                            const nesle_smb_shaped_params* params, void* state, float* reward, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NESLE_PPO_H */

/*
 * jointloom.h - C ABI of the MI355X (gfx950) hot path of JointLoom:
 * batched MAPF grid step, per-goal BFS fields, MAPF-GPT token builder,
 * MAGAT field-of-view + neighbour-graph builder.
 *
 * Plain C: device pointers, sizes and a HIP stream handle.  No torch types.
 * Every entry point enqueues its work on `stream` (a hipStream_t; NULL is the
 * legacy default stream) and returns 0 on success, a negative JL_ERR_* code
 * for an argument error detected on the host, or a positive hipError_t.
 * `jl_error_string` turns either into text.  No entry point synchronises the
 * stream or allocates device memory.
 *
 * Data layout (same bytes as the reference, /root/reference/src/cuda_backend):
 *   grid cell (x, y)   : flat index x*map_h + y, x = row in [0,map_w),
 *                        y = column in [0,map_h)          (grid_world_simulator.cpp:184-187)
 *   grid bitmap        : uint32 words, word = cell>>5, bit = cell&31,
 *                        map_w*map_h/32 words per env       (grid_world_cuda.h:17-23)
 *   agent state row    : 8 x uint16 {env, agent, pos_x, pos_y, target_x,
 *                        target_y, action, reset_flag}       (grid_world_cuda.h:129-138)
 *   MAPF-GPT raw row   : 13 x uint16 = state columns 0..7 + 5 history
 *                        actions (5 = empty)                 (mapf_gpt_schema.py:10-13,119-126)
 *   actions            : 0 wait, 1 (-1,0), 2 (+1,0), 3 (0,-1), 4 (0,+1)
 *                                                            (128_agents_map_step.cu:36-37)
 * Supported map profiles: map_h in {32, 64, 128, 256}, 1 <= map_w <= 256.
 */
#ifndef JOINTLOOM_H
#define JOINTLOOM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* jl_stream_t; /* hipStream_t */

/* int32 words of a MAPF-GPT builder's build_scratch (8320 bytes), and the
 * word that counts single-launch diagnostics waits that gave up (sticky; the
 * host reads and clears it). */
#define JL_BUILD_SCRATCH_WORDS 2080
#define JL_BUILD_SCRATCH_GAVE_UP_WORD 2

enum {
    JL_OK = 0,
    JL_ERR_ARG = -1,         /* null pointer, non-positive size, size overflow */
    JL_ERR_PROFILE = -2,     /* map_h not a multiple of 32 in [32, 256], or map_w outside [1, 256] */
    JL_ERR_CAPACITY = -3,    /* an edge buffer too small for the worst case */
    JL_ERR_AGENTS = -4       /* too many agents per env for a kernel's per-env LDS tables on
                                this map (the step: 2,048 agents per env on a 256x256 map
                                and about 2,280 with a fuller hash, more on smaller maps;
                                the token pass and the MAGAT passes allow more) */
};

/* Task modes (grid_world_cuda.h:44-46 of rebuttal/online-rl/native/src/cuda_backend):
 * lifelong goal resampling, standard MAPF with arrival latches and horizon,
 * and CostTracer (moves and step counts only; goals are advanced by
 * jl_costtracer_reward_goals). */
enum { JL_TASK_LIFELONG = 0, JL_TASK_STANDARD_MAPF = 1, JL_TASK_COSTTRACER = 2 };

/* Conflict outcome per agent and step (transition_adapters.py:361-455). */
enum {
    JL_OUTCOME_NONE = 0,
    JL_OUTCOME_WALL = 1,
    JL_OUTCOME_VERTEX = 2,
    JL_OUTCOME_SWAP = 3,
    JL_OUTCOME_CHAIN = 4
};

/* ------------------------------------------------------------------------ */
/* Simulator state (GridWorldContext, grid_world_cuda.h:47-97).  Every       */
/* pointer is device memory owned by the caller; [E,A] arrays are env-major. */
/* ------------------------------------------------------------------------ */
typedef struct jl_sim {
    int32_t n_envs;
    int32_t n_agents;
    int32_t map_w;
    int32_t map_h;
    int32_t task_mode;          /* JL_TASK_* */
    int32_t max_episode_steps;  /* horizon of standard_mapf */
    const uint32_t* grid_bits;  /* [E, W*H/32] static obstacles */
    uint32_t* grid_ocp;         /* [E, W*H/32] agent occupancy after the step */
    uint16_t* cur_x;            /* [E, A] */
    uint16_t* cur_y;            /* [E, A] */
    uint16_t* goal_x;           /* [E, A] */
    uint16_t* goal_y;           /* [E, A] */
    uint8_t* actions;           /* [E, A] action per agent; > 4 means wait */
    uint8_t* arrived;           /* [E, A] standard_mapf arrival latch */
    uint8_t* goal_changed;      /* [E, A] */
    float* rewards;             /* [E, A] 1.0 on goal after the step */
    uint8_t* terminated;        /* [E] */
    uint8_t* truncated;         /* [E] */
    int32_t* step_counts;       /* [E] */
    uint16_t* state_packed;     /* [E*A, 8] agent state rows */
    uint8_t* outcomes;          /* [E, A] JL_OUTCOME_* of the last step, or NULL */
    /* lifelong goal sampling (task_mode == JL_TASK_LIFELONG) */
    const uint32_t* free_cells; /* packed (x<<16|y), env-major, row-major per env */
    const int32_t* env_offsets; /* [E] first free cell of each env in free_cells */
    const int32_t* env_counts;  /* [E] number of free cells of each env */
    uint64_t* rng_state;        /* [E*A] per-agent generator state */
    /* Deterministic lifelong goals: when goal_candidates is not NULL, agents
     * on their goal take new goals in agent order from per-agent candidate
     * start lists instead of the generator (set_goal_candidates and the
     * canonical-order branch of rebuttal/online-rl/native/src/cuda_backend/
     * grid_world_simulator.cpp:901-918, 128_agents_map_step.cu:303-330). */
    const int32_t* goal_candidates;  /* [E, A, candidate_length] start indices */
    const uint16_t* candidate_cells; /* [E, candidate_stride, 2] (x, y) per env */
    const int32_t* candidate_counts; /* [E] cells of each env's list in use */
    int32_t* goal_cursors;           /* [E, A] goals taken so far (in/out) */
    int32_t candidate_length;
    int32_t candidate_stride;
} jl_sim_t;

/* Pack int32 [E, W, H] grids (nonzero = obstacle) into bitmaps.
 * Replaces launch_encode_full_map_kernel_on_stream, grid_world_cuda.cu:112-183. */
int jl_encode_map(const int32_t* grids, uint32_t* grid_bits, int32_t n_envs,
                  int32_t map_w, int32_t map_h, jl_stream_t stream);

/* One batched environment step with vertex / swap / chain conflict
 * resolution and standard-MAPF bookkeeping (or lifelong goal resampling).
 * Replaces launch_step_kernel, 128_agents_map_step.cu:25-377, called from
 * GridWorldSimulator::step_sim_only, grid_world_simulator.cpp:694-705. */
int jl_step(const jl_sim_t* sim, jl_stream_t stream);

/* Inclusive int64 prefix sum of the goal_changed values (uint8, summed as
 * int64) into prefix [E*A] and its total into count [1], on `stream` (no
 * host synchronisation).  A non-null changed_states (int16 [E*A, 8]) is
 * zero-filled for jl_energy_maps_flagged to pack into.  Replaces the cumsum,
 * count and fill of GridWorldSimulator::update_derived_state,
 * grid_world_simulator.cpp:709-733. */
int jl_goal_changed_scan(const jl_sim_t* sim, int64_t* prefix, int64_t* count,
                         uint16_t* changed_states, jl_stream_t stream);

/* Copy the caller's actions (uint8 [E, A], device memory) into the
 * simulator's action buffer on `stream`.  Replaces the device copy of
 * GridWorldSimulator::update_actions, grid_world_simulator.cpp:678-688. */
int jl_update_actions(const jl_sim_t* sim, const uint8_t* actions, jl_stream_t stream);

/* Point the action-reading kernels of an instantiated HIP graph at another
 * action buffer, without device work: every node of `graph` that is a
 * history append (jl_mapfgpt_append_actions) or an action copy
 * (jl_update_actions) reading `captured` reads `actions` in `graph_exec`
 * from its next launch on; *n_nodes (may be null) receives how many.
 * `actions` may have any alignment (the copy picks 16-byte words or bytes on
 * the device).  Every node is checked before any is changed.  No
 * counterpart in the reference, which launches every step from the host:
 * it serves graph replays of the resident loops (graphs.py), so that each
 * replay reads that step's actions where they lie instead of copying them
 * into the graph's buffer first. */
int jl_graph_retarget_actions(void* graph, void* graph_exec, const void* captured,
                              const void* actions, int32_t* n_nodes);

/* Write loaded positions/goals (int16 [E, A, 2] each), arrival latches
 * (uint8 [E, A]) and step counts (int32 [E]) into the simulator: split
 * state, terminated/truncated, zero rewards and actions, occupancy, packed
 * rows (reset_flag = 1), goals marked changed.  Inputs are trusted (the
 * caller validates them).  Replaces the device part of
 * GridWorldSimulator::load_state, grid_world_simulator.cpp:573-589, and
 * launch_load_state_kernel, 128_agents_map_step.cu:379-426. */
int jl_load_state(const jl_sim_t* sim, const int16_t* positions,
                  const int16_t* goals, const uint8_t* arrived,
                  const int32_t* step_counts, jl_stream_t stream);

/* Lifelong initialisation: free-cell lists and distinct random starts/goals.
 * `real_extents` is int32 [E, 2]; `free_cells` must hold E*W*H entries;
 * `env_offsets`/`env_counts` are written.  Replaces
 * cache_map_free_cells_kernel + init_agents_kernel, grid_world_cuda.cu:225-320,
 * 405-450, driven by run_initialization, grid_world_simulator.cpp:646-676. */
int jl_lifelong_init(const jl_sim_t* sim, const int32_t* real_extents,
                     uint32_t* free_cells, int32_t* env_offsets,
                     int32_t* env_counts, jl_stream_t stream);

/* Seed the per-agent generators (setup_rng_kernel, grid_world_cuda.cu:464-479). */
int jl_seed_rng(uint64_t* rng_state, int64_t count, uint64_t seed,
                jl_stream_t stream);

/* ------------------------------------------------------------------------ */
/* MAPF-GPT observation builder (MapfGPTCUDAContext, mapf_gpt_builder.h:8-21) */
/* ------------------------------------------------------------------------ */
typedef struct jl_mapfgpt {
    int32_t n_envs;
    int32_t n_agents;
    int32_t map_w;
    int32_t map_h;
    const uint32_t* grid_bits;  /* [E, W*H/32] */
    uint16_t* state_packed;     /* [N, 8] */
    uint16_t* histories;        /* [N, 5] */
    int64_t* labels;            /* [N] */
    uint16_t* cost_to_go;       /* [E, A, W, H] exact BFS distance, 0xFFFF unreachable,
                                   filled on request (jl_mapfgpt_cost_to_go); may be
                                   NULL for builds */
    int32_t* agent_at_cell;     /* [E, W, H] agent id or -1 (filled on request) */
    uint16_t* goal_cache;       /* [N, 2] goal of the last refresh (init 0xFFFF) */
    int32_t* tokens;            /* [N, 256] */
    uint8_t* active_mask;       /* [N] (torch.bool) */
    int32_t* diagnostics;       /* [4] overflow, bad row/action, duplicate cell, bad goal/position */
    uint32_t* agent_info;       /* [N] workspace: greedy-move mask and diagnostic flags of
                                   each agent, written by the first pass of a build */
    uint16_t* cost_tiles;       /* [E, A, ceil(W/8) + 2, H/8 + 2, 8, 8] workspace, 0xFFFF at
                                   allocation: the same fields as cost_to_go in 8x8 tiles
                                   (one 128-byte line per tile) inside a one-tile border of
                                   unreachable cells that no kernel writes; on maps of at
                                   most 4096 cells bits 12-15 of a reachable cell hold its
                                   greedy-move mask */
    int32_t* build_scratch;     /* [JL_BUILD_SCRATCH_WORDS] workspace, zero at construction,
                                   128-byte aligned, used with this builder's n_envs only:
                                   the single-launch build of small maps keeps in it the
                                   uint64 number of the last launch whose diagnostics were
                                   cleared, the count of diagnostics waits that gave up
                                   (word JL_BUILD_SCRATCH_GAVE_UP_WORD) and per-class
                                   workgroup arrival counters, from which each launch
                                   derives its number on the device (so builds captured
                                   into a graph keep one launch).  That number assumes the
                                   builds of one builder run one after another: issue them
                                   in order on one stream (or order the streams).  NULL =
                                   two-launch builds only */
    void* token_events[2];      /* optional hipEvent_t pair recorded on the stream right
                                   before / after the token kernel (profiling); NULL = off */
} jl_mapfgpt_t;

/* state_packed, cost_to_go, cost_tiles and tokens must be 16-byte aligned
 * (16-byte accesses) and build_scratch 128-byte aligned; the builds return
 * JL_ERR_ARG otherwise.
 *
 * cost_tiles holds the builder's fields; the token pass reads the windows
 * from it, and jl_mapfgpt_cost_to_go copies it into cost_to_go, so values
 * written into cost_to_go by the caller are not seen by later builds
 * (cost_to_go is an output).
 *
 * build_tokens(raw_rows int16 [N, 13]): unpack + goal-cache refresh + BFS of
 * refreshed goals + tokens.  Replaces MapfGPTObservationBuilder::build_tokens,
 * mapf_gpt_builder.cpp:89-114, and kernels mapf_gpt_cuda.cu:75-118, 181-325,
 * 328-347, 350-497. */
int jl_mapfgpt_build_rows(const jl_mapfgpt_t* b, const int16_t* raw_rows,
                          jl_stream_t stream);

/* jl_mapfgpt_build_rows for callers that cannot allocate (code under graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); it has no
 * counterpart in the reference.  It allocates nothing: instead of
 * b->build_scratch (ignored, may be NULL), it uses the library's own
 * 8320-byte per-device build scratch (a static device array, JL_BUILD_-
 * SCRATCH_WORDS words, that each device holds until the process ends).  One
 * fixed size serves every builder that jl_mapfgpt_build_rows accepts; larger
 * or malformed builders return JL_ERR_ARG / JL_ERR_PROFILE as there.  A
 * single-launch build first clears that scratch with a small kernel on
 * `stream` (two launches, no memset); a two-launch build does not use it.
 * Outputs equal jl_mapfgpt_build_rows's bit for bit.  All calls on one
 * device share its scratch: calls that overlap on one device (other streams,
 * other threads) race and must be serialised by the caller.  The count of
 * diagnostics waits that gave up is cleared with the scratch on every call
 * and is not reported.  `stream` must belong to the current device.  The
 * scratch's device address is looked up once per device and kept for the
 * life of the process: hipDeviceReset (which may move the array) is not
 * supported between calls. */
int jl_mapfgpt_build_rows_noalloc(const jl_mapfgpt_t* b, const int16_t* raw_rows,
                                  jl_stream_t stream);

/* build_tokens_from_state(cur_x, cur_y, goal_x, goal_y int16 [E, A]).
 * Replaces MapfGPTObservationBuilder::build_tokens_from_state,
 * mapf_gpt_builder.cpp:140-167, and mapf_gpt_state_unpack_kernel :121-152. */
int jl_mapfgpt_build_state(const jl_mapfgpt_t* b, const int16_t* cur_x,
                           const int16_t* cur_y, const int16_t* goal_x,
                           const int16_t* goal_y, jl_stream_t stream);

/* 1 when a build of this builder runs as one launch (maps of at most
 * 4096 cells with rows of at most 64 columns (map_h <= 64), an env of at
 * most 1024 agents, build_scratch set): unpack,
 * field refreshes and tokens of an env in one workgroup, also when captured
 * into a graph; 0 when it runs as two or three launches.  No
 * counterpart in the reference (a profiling query: the token_events pair
 * then brackets the whole build). */
int jl_mapfgpt_single_launch(const jl_mapfgpt_t* b);

/* Goal-cache refresh and BFS of changed goals from the resident split state,
 * without tokens: state rows, labels, goal cache, cost_to_go (and its tiled
 * copy), diagnostics [0] and [3].  Replaces
 * MapfGPTObservationBuilder::refresh_distances, mapf_gpt_builder.cpp:200-212 of
 * rebuttal/online-rl/native/src/cuda_backend. */
int jl_mapfgpt_refresh_state(const jl_mapfgpt_t* b, const int16_t* cur_x,
                             const int16_t* cur_y, const int16_t* goal_x,
                             const int16_t* goal_y, jl_stream_t stream);

/* append_actions(uint8 [E, A]).  Replaces mapf_gpt_append_actions_kernel,
 * mapf_gpt_cuda.cu:155-178. */
int jl_mapfgpt_append_actions(const jl_mapfgpt_t* b, const uint8_t* actions,
                              jl_stream_t stream);

/* reset_histories(): every history slot = 5 (mapf_gpt_builder.cpp:195-197). */
int jl_mapfgpt_reset_histories(const jl_mapfgpt_t* b, jl_stream_t stream);

/* Fill agent_at_cell from state_packed (the reference rewrites it on every
 * build, mapf_gpt_cuda.cu:328-347, 589-603; here it is filled on request). */
int jl_mapfgpt_agent_at_cell(const jl_mapfgpt_t* b, jl_stream_t stream);

/* Fill cost_to_go (row-major, plain distances) from the tiled fields the
 * builds keep.  The reference writes cost_to_go on every refresh
 * (mapf_gpt_cuda.cu:318-325); here refreshes write only the tiled copy and
 * the row-major one is filled on request. */
int jl_mapfgpt_cost_to_go(const jl_mapfgpt_t* b, jl_stream_t stream);

/* ------------------------------------------------------------------------ */
/* BFS distance fields                                                       */
/* ------------------------------------------------------------------------ */

/* uint8 "energy" fields for MAGAT: E = 255 - d for d <= 254, else 0, BFS
 * from each state row's target.  Rows whose env id is out of range are
 * skipped; with incremental_only only rows with reset_flag != 0 run.
 * `energy` is uint8 [E, A, W, H].  Replaces launch_energy_map_kernel,
 * energy_map.cu:80-272. */
int jl_energy_maps(const uint32_t* grid_bits, uint8_t* energy,
                   const uint16_t* states, int32_t length, int32_t n_envs,
                   int32_t n_agents, int32_t map_w, int32_t map_h,
                   int32_t incremental_only, jl_stream_t stream);

/* Stateful derived state: energy fields of every agent whose goal_changed
 * flag is set (all agents when `all_agents` != 0) from the simulator's goal
 * arrays.  Unless `all_agents`, each changed agent's state row (reset_flag 1)
 * is also written to changed_states[changed_prefix[g] - 1], where
 * changed_prefix is the inclusive int64 prefix sum of the flags
 * (pack_changed_agent_state_kernel, 128_agents_map_step.cu:469-511); when
 * its last value is 0 (no flag set) the launch returns at once.
 * Replaces GridWorldSimulator::update_derived_state,
 * grid_world_simulator.cpp:707-753, without its host synchronisation. */
int jl_energy_maps_flagged(const jl_sim_t* sim, uint8_t* energy,
                           int32_t all_agents, const int64_t* changed_prefix,
                           uint16_t* changed_states, jl_stream_t stream);

/* The incremental half of GridWorldSimulator::update_derived_state
 * (grid_world_simulator.cpp:707-753) in one call: jl_goal_changed_scan and
 * jl_energy_maps_flagged (all_agents 0) with the same outputs (prefix, count,
 * changed_states cleared and packed, energy fields of the changed agents),
 * as one launch for at most 131,072 agents on maps of at most 4,096 cells
 * and 64 rows, as the two launches otherwise.  changed_states may be NULL
 * (nothing packed). */
int jl_goal_changed_refresh(const jl_sim_t* sim, uint8_t* energy, int64_t* prefix, int64_t* count,
                            uint16_t* changed_states, jl_stream_t stream);

/* ------------------------------------------------------------------------ */
/* MAGAT builder (StatelessGridWorldContext, grid_world_cuda.h:99-117)        */
/* ------------------------------------------------------------------------ */
typedef struct jl_magat {
    int32_t n_envs;
    int32_t n_agents;
    int32_t map_w;
    int32_t map_h;
    const uint32_t* grid_bits;  /* [E, W*H/32] static obstacles */
    uint32_t* grid_ocp;         /* [E, W*H/32] agent occupancy */
    const uint8_t* energy;      /* [E, A, W, H] */
    const uint16_t* states;     /* [E*A, 8] rows the node builder reads */
    float* pyg_x;               /* [N, 4*13*13] */
    float* pyg_pos;             /* [N, 2] */
    int32_t* edge_counts;       /* [N] */
    int64_t* edge_prefix;       /* [N + 1] */
    int64_t* num_edges;         /* [1] */
    int64_t* edge_index;        /* [2, edge_capacity] */
    float* edge_attr;           /* [edge_capacity, 3] */
    int64_t edge_capacity;      /* >= E * A * (A - 1) */
    int64_t* env_edge_base;     /* [E + 1 + E * ceil(A / 64)] workspace: env bases, then
                                   the node builder's per-64-agent-slice edge totals */
} jl_magat_t;

/* Occupancy bitmap from agent state rows (rows with env id out of range are
 * ignored).  Replaces refresh_occ_bitmap_from_packed_states_kernel,
 * 128_agents_map_stateless_step.cu:140-173, 765-784. */
int jl_magat_occupancy(const jl_magat_t* m, jl_stream_t stream);

/* Node features pyg_x / pyg_pos and per-node edge counts.  Replaces
 * launch_materialize_pyg_nodes_from_packed_states,
 * 128_agents_map_stateless_step.cu:368-741. */
int jl_magat_nodes(const jl_magat_t* m, jl_stream_t stream);

/* Exclusive scan of edge counts, num_edges and COO edges ordered by source
 * then destination id.  Replaces launch_exclusive_scan_edge_counts,
 * grid_world_cuda.cu:17-110, and generate_pyg_edges_kernel,
 * 128_agents_map_stateless_step.cu:854-935. */
int jl_magat_edges(const jl_magat_t* m, jl_stream_t stream);

/* ------------------------------------------------------------------------ */
/* CostTracer (rebuttal/online-rl/native/src/cuda_backend/costtracer.{h,cu})  */
/* The simulator runs in JL_TASK_COSTTRACER mode; distances come from the     */
/* builder's fields after jl_mapfgpt_refresh_state (read from its tiled copy). */
/* best, cursor: int32 [E*A]; rewards, reached: float [E*A].                  */
/* ------------------------------------------------------------------------ */

/* Progress reward (0.1 when the distance to the goal fell below best), the
 * goal hit flag, and on a hit the next goal of the agent's stream
 * targets int16 [E, A, target_length, 2] (best becomes -1).  Replaces
 * costtracer_reward_goals / progress_goals, costtracer.cu:5-23, 87-103. */
int jl_costtracer_reward_goals(const jl_sim_t* sim, const jl_mapfgpt_t* b, int32_t* best,
                               const int16_t* targets, int32_t target_length,
                               int32_t* cursor, float* rewards, float* reached,
                               jl_stream_t stream);

/* Observation float [E*A, 2, 11, 11]: occupancy of the window around each
 * agent, and its distances normalised (cells without a distance placed 4
 * past the largest, shifted to 0, inverted and divided by the range), with
 * the progress feature -min(1, (d - best + 1) / 64) at the centre; best is
 * set to the agent's distance when negative or when its goal was refreshed.
 * Replaces costtracer_observe / observe, costtracer.cu:25-64, 105-113. */
int jl_costtracer_observe(const jl_sim_t* sim, const jl_mapfgpt_t* b, int32_t* best,
                          float* output, jl_stream_t stream);

/* Envs whose step count reached `horizon` start the next episode of the bank
 * (bank_positions/bank_goals int16 [bank_episodes, E, A, 2], episode =
 * ++episodes[e] % bank_episodes): positions, goals, occupancy, cursors 0,
 * best -1, step count 0.  Replaces costtracer_reset / reset_selected,
 * costtracer.cu:66-85, 115-127. */
int jl_costtracer_reset(const jl_sim_t* sim, const int16_t* bank_positions,
                        const int16_t* bank_goals, int32_t bank_episodes, int32_t* episodes,
                        int32_t* cursors, int32_t* best, int32_t horizon, jl_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Compact expert records (one stage = one joint step of every env)          */
/* ------------------------------------------------------------------------ */

/* A stage of compact records and the running state it is expanded against.
 * The full rows it stands for are the ones the reference's producers write
 * (mapf_gpt_online.py:215-258 with mapf_gpt_schema.py:43-66, 118-126 for 13
 * columns; topology_async.py:90-102, 235-278 for 8): env, agent, position,
 * goal, action, refresh flag (1 for every agent of an env whose episode starts
 * at this stage, else 0) and, for 13 columns, the 5 previous actions of the
 * running episode (oldest first, 5 = none).  `goals` and `history` carry the
 * running episode of every agent from one stage to the next; stages must be
 * expanded in order, and the first stage must start an episode in every env.
 * Device pointers; positions/goals 4-byte, history 8-byte aligned. */
typedef struct jl_records {
    int32_t n_envs;
    int32_t n_agents;
    int32_t features;               /* 8 or 13 */
    int32_t reserved;
    const uint16_t* positions;      /* [N, 2] x, y at this stage */
    const uint8_t* actions;         /* [N] action taken at this stage, 0..4 */
    const uint8_t* episode_start;   /* [E] 1 = env e starts an episode here */
    const uint16_t* new_goals;      /* [N, 2] goals; read for starting envs only */
    uint16_t* goals;                /* [N, 2] running goals (in/out) */
    uint8_t* history;               /* [N, 8] running histories, bytes 0..4 (in/out; 13 only) */
    int16_t* rows;                  /* out [N, features] */
} jl_records_t;

/* Rebuild one stage's rows of a frozen archive from its compact records
 * (the device side of RingStageSource streaming, frozen_stage_source.py:
 * 83-156; the rows equal the stages.npy rows save_records writes, :23-42). */
int jl_expand_records(const jl_records_t* r, jl_stream_t stream);

/* One step of the compact ring's DMA thread, on the host and `stream`
 * (CompactDMAWorker in the package): waits on the host for `staging_free`
 * (the staging buffer's previous upload), copies the stage's head (positions,
 * actions, start flags: 5N + E bytes) and the goal range of the envs that
 * start an episode from `host_slot` into the pinned `staging` buffer, uploads
 * them into `device_slot`, re-records `staging_free`, makes the stream wait
 * for `rows_free` (the consumer's copy out of the rows), expands the stage
 * into `records.rows` and records `done`.  Slot layout: positions [0, 4N),
 * actions [4N, 5N), start flags [5N, 5N + E), goals at the next multiple of
 * 16, 4N bytes.  `records` carries the sizes, running goals/histories and
 * rows; its stage pointers are set from `device_slot`.  Unlike the other
 * entry points it blocks the calling thread on `staging_free` (host memory
 * reuse) - the device stream is never synchronised.  No reference
 * counterpart: the reference's DMA thread is Python (expert_running.py:
 * 463-531) and streams full rows. */
typedef struct jl_stage_upload {
    const uint8_t* host_slot;
    uint8_t* staging;
    uint8_t* device_slot;
    int64_t slot_bytes;
    void* staging_free;   /* hipEvent_t, required */
    void* rows_free;      /* hipEvent_t or NULL */
    void* done;           /* hipEvent_t or NULL */
    int64_t bytes_uploaded;  /* out: bytes copied to the device */
    jl_records_t records;
} jl_stage_upload_t;

int jl_ring_upload_compact(jl_stage_upload_t* upload, jl_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Misc                                                                      */
/* ------------------------------------------------------------------------ */

/* Legacy observation decode (decode_to_uint8_kernel, grid_world_cuda.cu:186-210):
 * out[b, c, r, col] = (obs[b*2*diam + c*diam + r] >> col) & 1. */
int jl_decode_to_uint8(const uint16_t* obs, uint8_t* out, int64_t n_batch,
                       int32_t diameter, jl_stream_t stream);

/* Text for a status code returned by any entry point. */
const char* jl_error_string(int code);

/* Library version string. */
const char* jl_version(void);

#ifdef __cplusplus
}
#endif

#endif /* JOINTLOOM_H */

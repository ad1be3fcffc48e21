/*
 * kgx: the KataGo network forward pass on AMD Instinct MI355X (gfx950), as a C ABI.
 *
 * The entry points replace, one for one, what katago-nn-burn's backend does behind katago-core's
 * `NeuralNet` trait (crates/katago-core/src/neuralnet/nninterface.rs:79-214), so that a thin FFI backend
 * can implement that trait over them and leave NNEvaluator and `katago-rs analysis` unchanged.
 * Plain pointers and sizes only. Every function returning int returns 0 on success and nonzero on error,
 * with the message available from kg_last_error() on the calling thread.
 *
 * Threading: kg_net objects are immutable after loading and may be shared between threads. A kg_handle is
 * used by one thread at a time (calls on one handle are serialized by a lock); different handles may run
 * concurrently. kg_forward and kg_get_output block the calling thread until the batch's outputs are on the
 * host, so callers run them on a helper thread when their own thread must not wait
 * (crates/katago-nn-burn/src/backend.rs:735-753).
 */
#ifndef KGX_H
#define KGX_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KG_PRECISION_F32 0  /* float operands, float accumulate (the f32 tier) */
#define KG_PRECISION_F16 1  /* float16 GEMM operands, float accumulate and float residual streams */
#define KG_PRECISION_BF16 2 /* bfloat16 GEMM operands, float accumulate and float residual streams */

#define KG_MAX_POLICY_SIZE 362 /* NNPos::MAX_NN_POLICY_SIZE for 19x19 */

typedef struct kg_net kg_net;
typedef struct kg_handle kg_handle;

/* Library version string. */
const char* kg_version(void);

/* The last error message of the calling thread ("" if none). */
const char* kg_last_error(void);

/* Number of visible GPUs. Replaces the device probing of `katago_nn_burn::device`
 * (crates/katago-nn-burn/src/lib.rs:238-248). */
int kg_device_count(int* count);

/* Makes `device` current for this thread and initializes its runtime; a no-op when already open.
 * Replaces NeuralNet::global_initialize (backend.rs:244-252). */
int kg_device_open(int device);

/* Parses a KataGo model file (binary or text floats, optionally gzip-compressed) from memory.
 * Replaces NeuralNet::load_model_file (backend.rs:277-293): like it, a non-empty expected_sha256 is rejected
 * ("expectedSha256 is not supported"), and a model version above 17 is an error. */
int kg_net_load(const void* model_bytes, size_t len, const char* expected_sha256, kg_net** out);
void kg_net_free(kg_net* net);

/* The ModelDesc fields the engine reads (NeuralNet::get_model_desc, backend.rs:296-298). */
typedef struct {
  char name[128];
  int model_version;
  int num_input_channels;       /* spatial features (22 for v8+) */
  int num_input_global_channels;/* 19 for v8+ */
  int num_input_meta_channels;  /* 192 for human-SL nets, else 0 */
  int num_policy_channels;      /* P */
  int num_value_channels;       /* 3 */
  int num_score_value_channels; /* S */
  int num_ownership_channels;   /* 1 */
  int trunk_num_channels;
  int trunk_num_blocks;
  long num_parameters;
  float post_process_params[7]; /* td score, score mean, score stdev, lead, variance time, st value err, st score err */
  int output_row_len;           /* P*362 + 3 + S + 361 floats per row of kg_forward's output */
} kg_model_desc;
int kg_net_desc(const kg_net* net, kg_model_desc* out);

/* NNModelVersion::getInputsVersion / getNumSpatialFeatures / getNumGlobalFeatures
 * (crates/katago-core/src/neuralnet/modelversion.rs:40-110): the input layout of a model version (3..17).
 * Other versions fail with "NNModelVersion: Model version not currently implemented or supported: <v>".
 * Any output pointer may be NULL. */
int kg_model_version_features(int model_version, int* inputs_version, int* num_spatial, int* num_global);

/* NNModelVersion::getNumInputMetaChannels (modelversion.rs): 0 for meta encoder version 0, 192 for 1; other
 * versions fail with "NNModelVersion: metaEncoderVersion not currently implemented or supported: <v>". */
int kg_meta_encoder_channels(int meta_encoder_version, int* num_meta);

/* A device replica of the network with its own stream and workspace for up to max_batch rows.
 * Replaces create_compute_context + create_compute_handle (backend.rs:300-390) with their checks:
 * nn_x_len and nn_y_len must be 19 ("nnXLen and nnYLen must equal the network's posLen 19"), and
 * inputs_use_nhwc must be 0 ("inputsUseNHWC = true unsupported"); and the input buffers' check
 * (BurnInputBuffers::new, backend.rs:184-188): the model's input channel counts must be its version's.
 * precision is a KG_PRECISION_*. */
int kg_handle_create(const kg_net* net, int device, int max_batch, int precision, int nn_x_len, int nn_y_len,
                     int inputs_use_nhwc, kg_handle** out);
void kg_handle_free(kg_handle* handle);

/* Batch-shape buckets (BurnNeuralNet::with_batch_buckets, backend.rs:70-78): a batch of n rows runs as the
 * smallest bucket in [n, max_batch] (padded_batch_size, backend.rs:82-84); padding rows hold stale inputs.
 * Buckets <= 0 are dropped; count 0 clears them. */
int kg_handle_set_batch_buckets(kg_handle* handle, const int* buckets, int count);
int kg_padded_batch_size(const int* buckets, int count, int n, int max_batch);

/* Symmetry copy of one row of `channels` planes of h x w floats, NCHW (copy_with_symmetry,
 * crates/katago-core/src/neuralnet/nninputs.rs:756-850): symmetry bit 0 flips y, bit 1 flips x, bit 2
 * transposes (square planes only). reverse = 0 is copy_inputs_with_symmetry (nninputs.rs:872-874: a transpose
 * swaps the flips), reverse = 1 copy_outputs_with_symmetry (nninputs.rs:877-879). kg_get_output applies it to
 * the rows it stages and reads back. Host only; src and dst must not overlap. */
int kg_copy_with_symmetry(const float* src, float* dst, int channels, int h, int w, int symmetry, int reverse);

/* Whether the handle computes its GEMMs in a 16-bit type (NeuralNet::is_using_fp16, backend.rs:400-404). */
int kg_handle_is_using_fp16(const kg_handle* handle);

/* One forward pass of n rows (run_network, backend.rs:549-619): bin [n][C][19][19] NCHW float (after
 * symmetry), global [n][G], meta [n][192] or NULL when the net takes none. Writes n rows of
 * output_row_len floats: policy P x 362 (pass logit last in each channel), value 3, score S, ownership 361,
 * all raw (no softmax / tanh), in the order of the reference's concatenated readback (backend.rs:588-597). */
int kg_forward(kg_handle* handle, int n, const float* bin, const float* global, const float* meta, float* out);

/* The handle's device input and output buffers (max_batch rows each, layouts as in kg_forward). A caller that
 * fills them on the device can run kg_run without any host copy of the inputs. */
int kg_handle_device_buffers(kg_handle* handle, float** bin, float** global, float** meta, float** out);

/* The forward pass on the inputs already in the handle's device buffers. With out != NULL, also reads the n
 * output rows back to `out` and waits for them; with out == NULL, only enqueues the work on the handle's stream
 * (kg_sync waits). */
int kg_run(kg_handle* handle, int n, float* out);
int kg_sync(kg_handle* handle);

/* kg_run (out = NULL) without any allocation. No counterpart in the reference: it is for callers that cannot
 * allocate device memory, such as code under HIP graph capture, tight serving loops and harnesses that forbid
 * allocation. The forward pass runs on the inputs in the handle's device buffers and leaves its rows in the
 * handle's device output buffer (kg_handle_device_buffers), enqueued on the handle's stream without waiting
 * (kg_sync waits), as eager kernel launches only: no graph capture of its own, no event, no allocation. Its whole
 * workspace (activations and per-row partial results) is one static device array of 64 MiB per GPU, shared by
 * every call on that GPU and keeping the last call's contents: calls that overlap on one GPU, from any handle,
 * race and must be ordered by the caller. The first call on a handle looks the array up on the handle's device
 * and plans the forward pass for the largest batch up to max_batch whose workspace fits (host work only, no
 * device allocation); make that first call outside any stream capture. A batch whose workspace does not fit is
 * rejected with an error that names the capacity. */
int kg_run_static(kg_handle* handle, int n);

/* The handle's stream (a hipStream_t), for callers that order their own device work after kg_run. */
void* kg_handle_stream(kg_handle* handle);

/* Per-row inputs of get_output (NNResultBuf fields read by copy_inputs, backend.rs:497-546). */
typedef struct {
  const float* row_spatial; /* [C][19][19] NCHW, before symmetry */
  const float* row_global;  /* [G] */
  const float* row_meta;    /* [192] or NULL */
  int symmetry;             /* 0..7: bit 0 flipY, bit 1 flipX, bit 2 transpose */
  float policy_optimism;
} kg_row_input;

/* NNOutput fields written by copy_outputs (backend.rs:622-731). white_owner_map may be NULL. */
typedef struct {
  float policy_probs[KG_MAX_POLICY_SIZE];
  float white_win_prob, white_loss_prob, white_no_result_prob;
  float white_score_mean, white_score_mean_sq, white_lead, var_time_left;
  float shortterm_winloss_error, shortterm_score_error;
  float* white_owner_map; /* [361] or NULL */
} kg_nn_output;

/* NeuralNet::get_output (backend.rs:410-464): copy_inputs (symmetry per row), the forward pass (padded to a
 * bucket), one readback, copy_outputs (policy optimism mix, inverse symmetry, value / score unpacking by model
 * version). n must be in [1, max_batch]. */
int kg_get_output(kg_handle* handle, int n, const kg_row_input* rows, kg_nn_output* outputs);

/* get_output with the readback on a helper thread (backend.rs:598-605 and read_on_helper_thread,
 * backend.rs:743-753): copy_inputs runs on the calling thread (the rows are read before the call returns), the
 * uploads, the forward pass and one readback are enqueued, and the call returns; a helper OS thread then waits for
 * the device, runs copy_outputs into `outputs` and calls done(user, status) when done is not NULL (status 0 on
 * success). `outputs` (and their owner maps) must stay valid until then. `done` runs on the helper thread and must
 * not call functions on this handle (they would wait for that same thread). The next call on the handle, kg_wait
 * included, first waits for that thread; kg_wait also returns the helper's status, with its message in
 * kg_last_error() on failure. When the call itself fails, nothing was enqueued and `done` is not called. */
typedef void (*kg_done_fn)(void* user, int status);
int kg_get_output_async(kg_handle* handle, int n, const kg_row_input* rows, kg_nn_output* outputs, kg_done_fn done,
                        void* user);
int kg_wait(kg_handle* handle);

/* NNEvaluator's per-row inputs of the output post-processing (crates/katago-core/src/neuralnet/nneval.rs:1197-1500)
 * that come from the board, the rules and MiscNNInputParams. The legality of each move needs the rules engine and
 * stays with the caller: legal[i] is history.is_legal for NN position i (pass last), with any dagger-hack ban
 * (nneval.rs:1213-1222) already cleared. */
typedef struct {
  const unsigned char* legal;   /* [362], nonzero where the move is legal; at least one */
  int white_to_move;            /* nextPlayer == P_WHITE: the net's outputs are the mover's, flipped to white's */
  int board_x_size, board_y_size; /* board.x_size / y_size, 1..19 */
  float nn_policy_temperature;  /* MiscNNInputParams::nnPolicyTemperature (> 0) */
  int enable_passing_hacks;     /* MiscNNInputParams::enablePassingHacks: pass prior capped at 19x the rest */
  int no_result_allowed;        /* 0 when koRule != KO_SIMPLE and scoringRule != SCORING_TERRITORY */
} kg_post_input;

/* get_output (backend.rs:410-464) followed by NNEvaluator's post-processing of the fields (nneval.rs:1197-1500),
 * with copy_outputs and the post-processing on the device: the policy softmax over the legal moves at the
 * row's temperature (illegal moves -1), the value softmax, the score and error transforms by model version
 * (the version 3 arctan path included), and tanh ownership from white's perspective with 0 off the board. One
 * readback of the finished fields per batch. A nonfinite policy sum or value fails with the reference's
 * messages ("Got nonfinite for policy sum", "Got nonfinite for nneval value"). post has n entries. */
int kg_get_output_eval(kg_handle* handle, int n, const kg_row_input* rows, const kg_post_input* post,
                       kg_nn_output* outputs);

/* The same post-processing on n raw rows given on the host (kg_forward / kg_run layout), with each row's
 * symmetry and policy optimism: copy_outputs plus NNEvaluator's arithmetic, on the handle's device. */
int kg_post_outputs(kg_handle* handle, int n, const float* raw, const int* symmetry, const float* policy_optimism,
                    const kg_post_input* post, kg_nn_output* outputs);

/* copy_outputs alone (backend.rs:622-731), on the host: n raw rows of P*362 + 3 + S + 361 floats (kg_forward /
 * kg_run output) to NNOutput fields, with each row's symmetry (0..7) and policy optimism. For callers that run
 * the forward pass with kg_run on device-filled inputs. S must be the model version's score channel count. */
int kg_copy_outputs(const float* raw, int n, int num_policy_channels, int num_score_value_channels,
                    int model_version, const int* symmetry, const float* policy_optimism, kg_nn_output* outputs);

/* Kernel timing, for benchmarks: while enabled, kg_run / kg_forward launch eagerly and bracket every kernel
 * with events on the handle's stream. kg_profile_read reports, per kernel class, the launch count, the
 * summed duration in milliseconds and the summed algorithmic work (flops and bytes as defined per class).
 * Returns the number of classes (at most max_classes are written); names are static strings. */
int kg_profile_enable(kg_handle* handle, int enable);
int kg_profile_reset(kg_handle* handle);
int kg_profile_read(kg_handle* handle, const char** names, long* launches, double* ms, double* flops,
                    double* bytes, int max_classes);

/* A position for the device featurizer: the board, and the results of the rules engine (board history, ladder
 * search, area) that NNInputs::fill_row_v7 reads (crates/katago-core/src/neuralnet/nninputs.rs:1336-1800). Points
 * are indexed x + y * x_size (0 <= x < x_size, 0 <= y < y_size); colours and players are 0 empty, 1 black, 2 white.
 * The caller applies fill_row_v7's history rules: history_turns is min(maxTurnsOfHistoryToInclude,
 * numApproxValidTurnsThisPhase) as fill_row_v7 computes them (0 when a pass would end the game and it hides the
 * history), and pass_would_end_phase is 0 where it suppresses that feature. */
typedef struct {
  int x_size, y_size;              /* board size, 1..19 (at most the layout's) */
  int next_player;                 /* the player to move (1 or 2) */
  int ko_loc;                      /* Board::ko_loc, or -1 */
  int encore_phase;                /* hist.encore_phase: 0, 1 or 2 */
  int ko_rule;                     /* Rules::KO_SIMPLE 0, KO_POSITIONAL 1, KO_SITUATIONAL 2, KO_SPIGHT 3 */
  int scoring_rule;                /* Rules::SCORING_AREA 0, SCORING_TERRITORY 1 */
  int tax_rule;                    /* Rules::TAX_NONE 0, TAX_SEKI 1, TAX_ALL 2 */
  int multi_stone_suicide_legal;   /* hist.rules.multi_stone_suicide_legal */
  int has_button;                  /* hist.has_button */
  int pass_would_end_phase;        /* hist.pass_would_end_phase(board, next_player), or 0 where suppressed */
  int history_turns;               /* see above */
  int num_moves;                   /* entries of move_loc / move_player, most recent first, 0..5 */
  int move_loc[5];                 /* the move's point, -1 a pass, -2 Board::NULL_LOC */
  int move_player[5];
  float self_komi;                 /* hist.current_self_komi(next_player, drawEquivalentWinsForWhite) */
  double playout_doubling_advantage; /* MiscNNInputParams::playout_doubling_advantage */
  unsigned char color[361];        /* board.colors */
  unsigned char area[361];         /* the area colour: calculate_area (area scoring, no tax) or
                                    * calculate_independent_life_area, as fill_row_v7 chooses by the rules */
  unsigned char encore_start[361]; /* hist.second_encore_start_colors */
  unsigned char marks[361];        /* bit 0 hist.super_ko_banned, bit 1 hist.ko_recap_blocked, bits 2..5 the ladder
                                    * features 14..17 (iter_ladders over the board and the two previous boards) */
} kg_position;

/* The device featurizer: fill_row_v7 (nninputs.rs:1336-1800) for n positions, then copy_inputs' symmetry
 * (backend.rs:497-546, nninputs.rs:756-874), into the handle's device input buffers (the layout kg_run reads), on
 * the handle's stream, without waiting. The features that are functions of the board and the position's fields
 * (on-board, stones, liberties 1/2/3 by chain, ko, history, area, encore and ladder planes, the 19 globals) are
 * computed on the device. symmetry[i] in 0..7 (NULL: 0). The network must take the version-7 inputs (22 spatial, 19
 * global features: model versions 8 and up). Rejects a position whose fields are out of range, as the reference's
 * asserts would. A following kg_run (out != NULL) returns the rows. */
int kg_featurize(kg_handle* handle, int n, const kg_position* rows, const int* symmetry);

/* NNEvaluator's evaluation of n positions with everything between on the device: the featurizer (kg_featurize)
 * into the handle's input buffers, the forward pass (padded to a bucket), then get_output's copy_outputs and
 * NNEvaluator's post-processing (kg_get_output_eval), one readback of the finished fields. symmetry and
 * policy_optimism per row (NULL: 0 for every row); post and outputs as in kg_get_output_eval. The reference runs
 * these as three steps on the host around the backend (fill_row_bufs, nneval.rs:709-790; get_output,
 * backend.rs:410-464; the post-processing, nneval.rs:1197-1500). The network must take no metadata inputs. */
int kg_evaluate_positions(kg_handle* handle, int n, const kg_position* rows, const int* symmetry,
                          const float* policy_optimism, const kg_post_input* post, kg_nn_output* outputs);

/* The same featurizer with fill_row_v7's own layout arguments, between host buffers: bin gets n rows of 22 planes of
 * nn_x_len x nn_y_len (NCHW, or NHWC with use_nhwc), global n rows of 19, each after its symmetry (copy_inputs_with_
 * symmetry of the row; NULL: none). Runs on `device` and waits; allocates device memory for the call. */
int kg_featurize_rows(int device, int n, const kg_position* rows, int nn_x_len, int nn_y_len, int use_nhwc,
                      const int* symmetry, float* bin, float* global);

/* Launch geometry of the 16-bit implicit-GEMM convolution, for host-side checks of its index maps. No counterpart
 * in the reference (its convolutions are cubecl kernels with their own tiling, crates/katago-nn-burn/src/wino/
 * kernels.rs); these call the same functions as the kernel and its launcher, and launch nothing.
 * kg_conv_geometry: the configuration that a ks x ks convolution of ic -> oc channels (split: split operands, 1x1
 * only) over `pixels` pixels (batch x 361) runs. */
typedef struct {
  int grid;                /* workgroups launched */
  int threads;             /* threads per workgroup */
  int tile_rows, tile_cols;/* pixels and output channels per workgroup */
  int stage_channels;      /* input channels per K stage */
  int pixel_tiles, col_tiles;
  int pairs;               /* 1: 96-pixel tiles whose two halves of a 192-pixel tile share an XCD */
  int weights_direct;      /* 1: the stage's weights go from memory straight into LDS */
  int weight_rows;         /* weight rows per stage (taps x tile_cols) */
  int waves;               /* waves per workgroup */
  int direct_instructions; /* direct loads (8 rows of 128 bytes each) that fill one stage's weight rows */
  int direct_per_wave;     /* direct loads each wave issues per stage */
} kg_conv_geometry_t;
int kg_conv_geometry(int ks, int ic, int oc, int split, int pixels, kg_conv_geometry_t* out);
/* The (pixel tile, column tile) that workgroup `workgroup` computes; -1, -1 when it exits at once. */
int kg_conv_tile_of(int ks, int ic, int oc, int split, int pixels, int workgroup, int* pixel_tile, int* col_tile);
/* Weights straight into LDS: the weight row and 16-byte chunk that lane `lane` of wave `wave` reads with its
 * direct load q of a stage, and the LDS weight row and chunk it fills (dst_row -1: a spare area nothing reads). */
int kg_conv_weight_load(int ks, int ic, int oc, int split, int q, int wave, int lane, int* src_row, int* src_chunk,
                        int* dst_row, int* dst_chunk);
/* The stored chunk of logical 16-byte chunk `chunk` of LDS weight row `row` (what the fragment reads address). */
int kg_conv_weight_chunk(int row, int chunk);
/* The nested-bottleneck junction launch (one block's exit 1x1 convolution, 192 -> 384, and the next block's entry
 * 1x1, 384 -> 192, in one kernel) over `pixels` pixels: its workgroup count, and the 48-pixel tile that workgroup
 * `workgroup` computes (-1 when it exits at once). No counterpart in the reference: the index map its kernel uses,
 * for host-side checks. */
int kg_junction_tile_of(int pixels, int workgroup, int* grid, int* tile);
/* The gpool blocks' tile launch (a global-pooling block's mid activation per 192-pixel tile: pooled features,
 * row-bias matmul, emission) over `pixels` pixels for a block of gpool_channels pooled and regular_channels
 * regular channels: its workgroup count, the 192-pixel tile of workgroup `workgroup` (-1 when it exits at once) and
 * the regular channels it emits [first_channel, first_channel + channels). No counterpart in the reference: the
 * index map its kernel uses, for host-side checks. */
int kg_gpool_tile_of(int pixels, int gpool_channels, int regular_channels, int workgroup, int* grid, int* tile,
                     int* first_channel, int* channels);
/* The 128-byte line (of the next op's weights) that thread `thread` of workgroup `workgroup` of a `grid`-workgroup
 * launch touches into its XCD's L2 (workgroup g runs on XCD g mod 8; lines past the weights are not read). No
 * counterpart in the reference: the index map the kernels use, for host-side checks. */
int kg_l2_touch_line(int grid, int workgroup, int thread, int* line);
/* The transformer RMSNorm launch over `rows` token rows of `channels` channels, when the rows were written in row
 * tiles of `region` rows (tile r on XCD r mod 8; 0: no such tiles): its workgroup count, and the rows
 * [first_row, first_row + count) of workgroup `workgroup` (count 0 when it exits at once). No counterpart in the
 * reference: the index map its kernel uses, for host-side checks. */
int kg_rmsnorm_rows_of(int rows, int channels, int region, int workgroup, int* grid, int* first_row, int* count);

#ifdef __cplusplus
}
#endif

#endif /* KGX_H */

/* C ABI of the compiled inference executor in libmunet_hip.so.
 *
 * Mirrors inference::Engine (reference src/inference.hpp:292-801):
 *   load    -> mh_engine_create (module config) + mh_engine_set_param
 *              (reference Engine::load(module) / load_serialized,
 *              src/inference.hpp:389-444, src/inference_serialization.cpp:1086)
 *   compile -> mh_engine_compile (reference Engine::compile,
 *              src/inference.hpp:446-537: shape contract + warm-up forward).
 *              Here compile also traces the module tree into an op list,
 *              fuses epilogues (bias, ReLU/GELU, residual, head split,
 *              zero-copy concat), plans every activation into one hipMalloc
 *              arena by liveness, and captures the forward as a hipGraph.
 *   run     -> mh_engine_run (reference Engine::run, src/inference.hpp:
 *              541-610): H2D of the input, one graph launch, D2H of the output.
 *   stats   -> mh_engine_stats (EngineStats, src/inference.hpp:43-66) as JSON.
 *
 * Config JSON uses the reference's serialized module schema
 * (src/inference_serialization.cpp:762-860: Sequential, Linear, Conv2d,
 * MaxPool2d, Upsample, ReLU, Sigmoid, GELU, Softmax, Flatten, LayerNorm,
 * Embedding, MultiHeadAttention) plus the composite TransformerBlock,
 * DecoderLM and UNet workloads; "dtype" is float32 / float16 / bfloat16.
 * Parameter names follow Module::named_parameters (src/core/module.hpp:95-107).
 *
 * device < 0 creates a plan-only engine: compile traces, fuses and plans but
 * touches no GPU (used to test the planner on hosts without a GPU). */
#ifndef MUNET_HIP_ENGINE_H
#define MUNET_HIP_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mh_engine mh_engine;

int mh_engine_create(mh_engine **engine, const char *config_json, int device);
int mh_engine_destroy(mh_engine *engine);
/* Create an engine from a MuNet deploy artifact (`munet_model` rev-1 .npz:
 * `__config__` JSON + one .npy per named parameter), validating its metadata
 * as the reference loader does (reference inference::load_serialized,
 * src/inference_serialization.cpp:902-1080, plus Engine::load).  Tensors may
 * be <f4, <f2, <i4, or <u2 holding bf16 bit patterns; floating tensors are
 * converted to the config's dtype with MuNet's codecs. */
int mh_engine_create_from_artifact(mh_engine **engine, const char *path, int device);
/* Copy one parameter (host storage bits of `dtype`, MuNet layout) into the
 * engine; weights are packed for the kernels at compile time. */
int mh_engine_set_param(mh_engine *engine, const char *name, const void *host_data, size_t bytes, int dtype);
/* Compile for one input shape (exact shape contract). */
int mh_engine_compile(mh_engine *engine, const int *input_shape, int ndim);
/* Engine::load (src/inference.hpp:393-444): the parameters set so far are the
 * module; emits LoadStarted / LoadCompleted to the observer (the completion
 * message names the parameter count and bytes unless in lean mode).  Compile
 * loads first when the caller has not. */
int mh_engine_load(mh_engine *engine);
/* EngineConfig (src/inference.hpp:32-41; setters :311-335): warmup_runs >= 0
 * (compile runs warmup_runs - 1 graph forwards after its own first one,
 * reported as compile_warmup_ms); strict_shape_check = 0 lets a run with any
 * input shape compile its own instance instead of failing the contract;
 * lean_mode = 1 leaves memory figures and the parameter scan out of events.
 * Compile and run events carry a fresh trace id while an observer is
 * attached (EngineStats last_compile_trace_id / last_run_trace_id). */
int mh_engine_set_config(mh_engine *engine, int warmup_runs, int strict_shape_check, int lean_mode);
/* Device address of the input / output buffers inside the arena. */
int mh_engine_input_ptr(mh_engine *engine, void **ptr);
int mh_engine_output_ptr(mh_engine *engine, void **ptr);
/* Output shape (ndim written to *ndim, dims to shape[0..ndim)). */
int mh_engine_output_shape(mh_engine *engine, int *shape, int *ndim);
/* Host-to-host forward: input/output are host buffers in storage format. */
int mh_engine_run(mh_engine *engine, const void *host_input, void *host_output);
/* Forward on the device-resident input buffer; waits for completion. */
int mh_engine_run_device(mh_engine *engine);
/* Enqueue one forward (graph launch) on the engine stream without waiting. */
int mh_engine_launch(mh_engine *engine);
/* The engine's HIP stream. */
int mh_engine_stream(mh_engine *engine, void **stream);
/* EngineStats as a JSON object. */
int mh_engine_stats(mh_engine *engine, char *buf, size_t len);
/* ---- caller features of the reference Engine ----------------------------
 * Compile with an expected input shape whose -1 entries are wildcards
 * (reference Engine::compile(example, expected_input_shape) and ShapeContract,
 * src/inference.hpp:128-184, 446-537).  Runs on other shapes that satisfy the
 * contract compile one more graph instance per concrete shape on first use;
 * all instances share the weight arena. */
int mh_engine_compile_expected(mh_engine *engine, const int *example_shape, int ndim, const int *expected_shape);
/* Output shape for an input shape (compiles its instance if needed). */
int mh_engine_output_shape_for(mh_engine *engine, const int *input_shape, int ndim, int *out_shape, int *out_ndim);
/* Host-to-host forward for an input of the given shape (contract-checked). */
int mh_engine_run_shaped(mh_engine *engine, const void *host_input, const int *shape, int ndim, void *host_output);
/* Forward through the prepared-input cache (reference PreparedInputCache and
 * prepare_input, src/inference.hpp:186-289, 665-686): `key` identifies the
 * caller's input tensor and `version` its mutation count; a hit reuses the
 * device copy made on a miss. */
int mh_engine_run_cached(mh_engine *engine, const void *host_input, uint64_t key, uint64_t version,
                         void *host_output);
/* Cache capacity (EngineConfig prepared_input_cache_entries / _max_bytes,
 * defaults 8 and 64 MiB); clears the cache. */
int mh_engine_set_input_cache(mh_engine *engine, size_t max_entries, size_t max_bytes);
int mh_engine_clear_input_cache(mh_engine *engine);
/* run_batch_into (src/inference.hpp:618-627): n host inputs -> n host outputs. */
int mh_engine_run_batch(mh_engine *engine, int n, const void *const *host_inputs, void *const *host_outputs);
/* Observer (EngineObserver / EngineEvent, src/inference.hpp:68-94): called
 * with one JSON object per CompileStarted / CompileCompleted / RunStarted /
 * RunCompleted / Error event; NULL removes it. */
typedef void (*mh_engine_observer)(const char *event_json, void *user);
int mh_engine_set_observer(mh_engine *engine, mh_engine_observer fn, void *user);
/* Pinned host staging for the PCIe path: the engine's page-locked input and
 * output buffers (allocated on first call) and a forward between them. */
int mh_engine_pinned_io(mh_engine *engine, void **host_input, void **host_output);
int mh_engine_run_pinned(mh_engine *engine);
/* The compiled plan (ops, fused epilogues, arena offsets) as JSON. */
int mh_engine_plan(mh_engine *engine, char *buf, size_t len);
/* GPU time of every op of the compiled forward (or only the ops named
 * `only`, when not NULL or empty) on its own, as a JSON list of
 * {name, kind, us, flops, bytes} (us per launch over `reps` launches replayed
 * from one graph on the engine stream; flops / bytes: the op's algorithmic
 * work).  Per-op counterpart of the reference's module Profiler
 * (src/core/module.hpp:71-83, src/core/util/profiler.hpp). */
int mh_engine_op_times(mh_engine *engine, int reps, const char *only, char *buf, size_t len);
/* GPU time of every op inside the compiled forward, as the same JSON list:
 * for each prefix ops[0..i] of the forward, a graph of that prefix is
 * replayed `reps` times between events, and op i's time is the difference of
 * consecutive prefix times (the caches and transitions of the graph; op 0
 * also holds the graph launch overhead).  The in-graph side of the same
 * Profiler (src/core/module.hpp:71-83). */
int mh_engine_forward_op_times(mh_engine *engine, int reps, char *buf, size_t len);

/* ---- KV-cache decode --------------------------------------------------------
 * No counterpart in the reference: its roadmap lists a KV cache
 * (documentation/architecture/gpt3_local_roadmap.md:67) that the code does
 * not have, and its attention reads the keys through a reinterpretation of
 * k's buffer (src/nn/attention.hpp:64-67), so a position's key is not its
 * own and cannot be cached.  A decoder therefore runs DecoderLM configs with
 * "attention": "textbook" (key j of a head is position j's key; every
 * rounding step of the reference's chain kept), whose engine forward is the
 * prefill.  Greedy decoding: each step feeds one token per sequence. */
typedef struct mh_decoder mh_decoder;
/* A decoder over a compiled engine (weights shared with it), `batch`
 * sequences (1..16), positions 0..max_len-1 (max_len <= ctx, at most 4096);
 * head_dim a multiple of 8 and at most 64, d_model and ffn rows multiples of
 * 16 bytes, batch x max(d_model, ffn) values within 64 KiB. */
int mh_decoder_create(mh_decoder **decoder, mh_engine *engine, int batch, int max_len);
int mh_decoder_destroy(mh_decoder *decoder);
/* Prompt ids [batch, T0] (int32) through the engine's forward, filling the
 * caches for positions 0..T0-1; logits_out [batch, T0, vocab] (storage
 * dtype) optional.  The next step's input becomes each sequence's greedy
 * choice at position T0-1. */
int mh_decoder_prefill(mh_decoder *decoder, const int32_t *ids, int T0, void *logits_out);
/* One step at the next position: ids [batch] (NULL: the previous greedy
 * choices); logits_out [batch, vocab] and next_ids [batch] optional. */
int mh_decoder_step(mh_decoder *decoder, const int32_t *ids, void *logits_out, int32_t *next_ids);
/* n greedy steps back to back (one graph launch each): tokens_out [n, batch];
 * gpu_ms (optional): device time of the n steps. */
int mh_decoder_generate(mh_decoder *decoder, int n, int32_t *tokens_out, float *gpu_ms);
/* The position the next step feeds (-1 before the first prefill). */
int mh_decoder_position(mh_decoder *decoder, int *pos);
/* Sizes, step count and last timings as JSON. */
int mh_decoder_stats(mh_decoder *decoder, char *buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* MUNET_HIP_ENGINE_H */

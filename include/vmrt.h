/*
 * vmrt.h -- C ABI of the MI355X megakernel VM runtime (libvmrt.so).
 *
 * This is the thin native layer that the Python lowering/scheduler and the PJRT
 * plugin drive: it owns HIP device buffers, the per-program arena and the
 * persistent-kernel launch.  Every entry point is plain C (pointers, sizes,
 * integer status codes) so any FFI can bind it (ctypes, cgo, JNI, N-API).
 *
 * Each function names the reference interface it replaces
 * (/root/reference/pjrt_plugin/src/runtime.h unless noted).
 *
 * Status codes follow PJRT_Error_Code numbering (pjrt_c_api.h), which is what the
 * reference's PJRT layer maps its runtime failures to (plugin.cc:588-592,
 * 632-637, 754-761, 784-790, 944-972).
 */
#ifndef VMRT_H_
#define VMRT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  VMRT_OK = 0,
  VMRT_INVALID_ARGUMENT = 3,
  VMRT_NOT_FOUND = 5,
  VMRT_RESOURCE_EXHAUSTED = 8,
  VMRT_FAILED_PRECONDITION = 9,
  VMRT_UNIMPLEMENTED = 12,
  VMRT_INTERNAL = 13,
  VMRT_UNAVAILABLE = 14,
};

typedef struct vmrt_runtime vmrt_runtime;
typedef struct vmrt_program vmrt_program;
typedef struct vmrt_launch vmrt_launch;

typedef struct {
  int32_t device;              /* HIP device ordinal */
  uint32_t n_lanes;            /* 0: one lane per compute unit */
  uint32_t ew_ts;              /* elements per EW tile; 0: 4096 */
  uint32_t mma_t;              /* default MMA output tile edge; 0: 128 */
  uint32_t cooperative;        /* 1: cooperative launch; 0 (default via 0xFFFFFFFF): plain */
  uint32_t barrier_timeout_ms; /* grid-barrier wait limit; 0: 2000 ms */
} vmrt_options;

typedef struct {
  uint32_t n_lanes;          /* lanes a program may be scheduled for */
  uint32_t max_lanes;        /* co-resident lane limit (CUs x occupancy) */
  uint32_t ew_ts;
  uint32_t mma_t;
  uint32_t compute_units;
  uint32_t lanes_per_cu;
  uint32_t lds_bytes;        /* LDS used per lane */
  uint32_t cooperative;
  char arch[64];             /* gcnArchName */
  char name[128];
} vmrt_device_info;

/* Fill `opts` with defaults (device 0, everything else chosen at create). */
void vmrt_default_options(vmrt_options* opts);

/* Open a device and prepare the VM kernel.
 * Replaces OclRuntime::Create (runtime.h:120-135; runtime.cc:255-662). */
int vmrt_create(const vmrt_options* opts, vmrt_runtime** out, char* err, size_t errlen);

/* Replaces OclRuntime::~OclRuntime.  Waits for the runtime's stream and for each
 * loaded program's latest launch on the stream it was enqueued on (which must
 * still exist; other work on the device is not waited for), then unloads every
 * program still loaded on this runtime (a program borrows its runtime's device,
 * stream and mutex, runtime.h:365): their handles are invalid afterwards and must
 * not be passed to vmrt_unload or any other call.  Launch handles of
 * vmrt_submit must be released before. */
void vmrt_destroy(vmrt_runtime* rt);

/* Device parameters the lowering must schedule for: these are the values the
 * reference hands the lowering subprocess as PJRT_OCL_NLANES / _EW_TS / _MMA_T
 * (plugin.cc:770-780; OclRuntime::ngroups/ew_ts/mma_t accessors, runtime.h). */
int vmrt_device_info_get(vmrt_runtime* rt, vmrt_device_info* out);

/* Parse, validate and load a VMProgram v3 blob: arena, constants, tasks,
 * entries, lane table, aux pool; buffer ids patched to handles.
 * Replaces VmProgram::Parse + LoadedProgram::Load (runtime.h:300-352;
 * runtime.cc:90-251, 735-1074).  ew_ts / mma_t of 0 use the runtime's values; they
 * must equal what the program was scheduled with. */
int vmrt_load(vmrt_runtime* rt, const void* bytes, size_t len, uint32_t ew_ts, uint32_t mma_t,
              vmrt_program** out, char* err, size_t errlen);

/* Replaces LoadedProgram::~LoadedProgram (runtime.cc:1076-1086).  Waits for the
 * program's latest launch first, on the stream it was enqueued on (which must
 * still exist). */
void vmrt_unload(vmrt_program* prog);

/* Program signature (executable metadata the PJRT layer reports,
 * plugin.cc:792-806): counts, then per input / output index its dtype (VMProgram
 * dtype enum), byte size, rank and dims (up to 16). */
int vmrt_program_counts(vmrt_program* prog, uint32_t* n_inputs, uint32_t* n_outputs, uint32_t* n_lanes);
int vmrt_program_io(vmrt_program* prog, int is_output, uint32_t index, uint32_t* dtype, uint64_t* bytes,
                    uint32_t* rank, uint64_t* dims16);

/* Run the program on device buffers: inputs are read in place and outputs
 * written in place (zero-copy ports), then wait for completion and check the VM
 * status word.  Replaces LoadedProgram::ExecuteDevice (runtime.h:340-346;
 * runtime.cc:2107-2242). */
int vmrt_execute(vmrt_program* prog, const void* const* inputs, size_t n_inputs, void* const* outputs,
                 size_t n_outputs, char* err, size_t errlen);

/* Same, asynchronously on `stream` (a hipStream_t; NULL = the runtime's stream).
 * No completion wait and no status check: call vmrt_program_status after
 * synchronizing.  Calls that overlap on one program share its arena and race. */
int vmrt_enqueue(vmrt_program* prog, const void* const* inputs, size_t n_inputs, void* const* outputs,
                 size_t n_outputs, void* stream, char* err, size_t errlen);

/* Parse, validate and run a VMProgram v3 blob once, synchronously, without
 * allocating: no hipMalloc / hipFree and no allocating library routine.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc).  It is not for
 * use under HIP graph capture: it uploads the program's tables with copies on
 * the runtime's stream and synchronizes that stream before it returns.  The
 * program's arena, side tables, barrier words and task
 * scratch live in a static device array of 64 MiB per GPU, reserved when the
 * library loads and held until the process ends; a program needing more is
 * rejected with VMRT_RESOURCE_EXHAUSTED.  Inputs and outputs are the caller's
 * device buffers, as for vmrt_execute (same results).  Every call on one GPU
 * shares that GPU's array and clears what must start at zero; calls through one
 * runtime serialise on its mutex, while overlapping calls on one GPU through
 * different runtimes race. */
int vmrt_run_noalloc(vmrt_runtime* rt, const void* bytes, size_t len, uint32_t ew_ts, uint32_t mma_t,
                     const void* const* inputs, size_t n_inputs, void* const* outputs, size_t n_outputs, char* err,
                     size_t errlen);

/* One launch with a status of its own, for callers with several launches of
 * one program in flight (the PJRT plugin's asynchronous Execute).  Enqueues the
 * program on the runtime's stream as vmrt_enqueue does, followed by a status
 * epilogue that copies the VM status word into a slot of pinned host memory
 * owned by this launch and, when the launch aborted, clears the program's
 * control words and task scratch, so a launch queued behind it starts clean.
 * vmrt_launch_query returns VMRT_OK once the launch and its epilogue have
 * completed and VMRT_UNAVAILABLE while they have not, without waiting and
 * without taking the runtime's lock; vmrt_launch_wait waits for them and returns
 * this launch's own outcome (VMRT_INTERNAL with the VM's message when it
 * aborted).  vmrt_launch_release waits for the launch and frees the handle.  No
 * counterpart in the reference, whose execution is synchronous
 * (plugin.cc:175-184, runtime.cc:2185-2189).  The program's shared status word
 * is left clear, so vmrt_program_status does not report a submitted launch. */
int vmrt_submit(vmrt_program* prog, const void* const* inputs, size_t n_inputs, void* const* outputs,
                size_t n_outputs, vmrt_launch** out, char* err, size_t errlen);
int vmrt_launch_query(vmrt_launch* launch);
int vmrt_launch_wait(vmrt_launch* launch, char* err, size_t errlen);
void vmrt_launch_release(vmrt_launch* launch);

/* Wait for the stream of the program's latest launch (the runtime's, or the
 * stream given to vmrt_enqueue, which must still exist), then read and clear
 * the program's VM status
 * word (barrier time-out, frame overflow).  Extension of the reference, whose
 * clFinish error path only reports an OpenCL code (runtime.cc:2185-2189). */
int vmrt_program_status(vmrt_program* prog, char* err, size_t errlen);

/* Per-task profile of the executions since the last reset, when the program was
 * loaded with PJRT_AMD_PROFILE=1 (FAILED_PRECONDITION otherwise).  Fills
 * 4 + 4 * n_tasks words, in 100 MHz ticks: [0] lane-time spent in grid barriers,
 * [1] lane-barriers, [2] lane-time from launch start to each lane's end, [3]
 * lane-time waiting for completion flags; task i at 4 + 4 i: lane-time summed
 * over its entries, the longest single entry, the entry count.  Replaces the reference's per-phase
 * profiling queue (PJRT_OCL_PROFILE, runtime.cc:2122-2195). */
int vmrt_program_profile(vmrt_program* prog, uint64_t* out, size_t n_words, int reset, char* err, size_t errlen);

/* Device memory through the runtime's size-bucketed pool.
 * Replace OclRuntime::AllocDevice / PoolAlloc / PoolFree (runtime.h:229-262;
 * runtime.cc:2244-2273). */
int vmrt_alloc(vmrt_runtime* rt, size_t bytes, void** dptr, char* err, size_t errlen);
int vmrt_free(vmrt_runtime* rt, void* dptr);

/* Blocking copies.  Replace OclRuntime::WriteToDevice / ReadFromDevice
 * (runtime.h:264-272; runtime.cc:2279-2301); d2d is the arena copy of
 * ExecuteDevice (runtime.cc:2135-2146, 2174-2184). */
int vmrt_h2d(vmrt_runtime* rt, void* dst, const void* src, size_t bytes, char* err, size_t errlen);
int vmrt_d2h(vmrt_runtime* rt, void* dst, const void* src, size_t bytes, char* err, size_t errlen);
int vmrt_d2d(vmrt_runtime* rt, void* dst, const void* src, size_t bytes, char* err, size_t errlen);

/* Wait for all work on the runtime's stream. */
int vmrt_synchronize(vmrt_runtime* rt, char* err, size_t errlen);

/* The runtime's hipStream_t (for callers that time or order work around it). */
void* vmrt_stream(vmrt_runtime* rt);

/* HIP events for timing work on a stream (NULL stream = the runtime's).  The
 * reference times with OpenCL profiling queues (PJRT_OCL_PROFILE,
 * runtime.cc:2122-2195); these give callers the same device-side clock. */
int vmrt_event_create(vmrt_runtime* rt, void** event);
int vmrt_event_record(vmrt_runtime* rt, void* event, void* stream);
int vmrt_event_elapsed_ms(void* start, void* stop, float* ms);
void vmrt_event_destroy(void* event);

/* Completion of the work recorded before `event`: vmrt_event_query returns
 * VMRT_OK once it has completed and VMRT_UNAVAILABLE while it has not;
 * vmrt_event_synchronize waits for it.  VMRT_INTERNAL on a HIP error.  With
 * vmrt_enqueue these give the asynchronous execution the reference's events
 * stand for (plugin.cc:175-184, where every event is born complete). */
int vmrt_event_query(void* event);
int vmrt_event_synchronize(void* event);

/* Measure the scheduler's cost table on this device and write it as one JSON
 * object into `json` (cap bytes): per-tile microseconds of the elementwise,
 * matmul, reduce and gather tile ops on one lane ("ew_tile_us", "mma_tile_us",
 * "reduce_tile_us", "gather_tile_us", the reference's keys), and the terms of
 * this build's phase model: "tile_us" (a tile's latency), "lane_gbs" (per-lane
 * streaming GB/s with every lane streaming), "barrier_us" and
 * "barrier_us_per_lane" (the grid barrier's cost at L lanes is
 * barrier_us + barrier_us_per_lane * L), "lane_mma_tflops".  Takes tens of
 * milliseconds.  Replaces OclRuntime::CalibrateCosts (runtime.cc:2433-2517;
 * the table the lowering reads through PJRT_OCL_COST_TABLE, plugin.cc:770-780). */
int vmrt_calibrate(vmrt_runtime* rt, char* json, size_t cap, char* err, size_t errlen);

/* Library version string. */
const char* vmrt_version(void);

#ifdef __cplusplus
}
#endif

#endif /* VMRT_H_ */

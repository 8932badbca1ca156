// Structures shared by the host runtime (vmrt.cpp) and the persistent VM kernel
// (vm_kernel.hip).  Field layouts are the VMProgram v3 schedule sections
// (reference: python/pjrt_ocl/scheduler.py:99-106,226-248;
// pjrt_plugin/src/runtime.h:20-104), so the loader can upload them verbatim after
// patching buffer ids to handles.
#pragma once
#include <stdint.h>

namespace vm {

// ---- element types (lowering.py:59-81) ------------------------------------------
enum Dtype : uint32_t {
  DT_F32 = 0, DT_I32 = 1, DT_U32 = 2, DT_BOOL = 3,
  DT_I64 = 4, DT_F64 = 5, DT_F16 = 6, DT_BF16 = 7, DT_COUNT = 8
};

// ---- tile ops (scheduler.py:47-71) -----------------------------------------------
enum TileOp : uint32_t {
  TOP_EW = 0, TOP_MMA = 1, TOP_GATHER = 2, TOP_RED_PART = 3, TOP_RED_COMB = 4,
  TOP_IOTA_DIM = 5, TOP_SCATTER = 6, TOP_DYN_GATHER = 7, TOP_DYN_SCATTER = 8,
  TOP_RED_WINDOW = 9, TOP_RED_SEG = 10, TOP_SOFTMAX_SEG = 11,
  TOP_LAYERNORM_SEG = 12, TOP_MAP_REGION = 13, TOP_FLASH_ATTN = 14,
  TOP_RED_STRIDED = 15, TOP_GATHER_INDEX = 16, TOP_CONV = 17,
  TOP_SCATTER_INDEX = 18,
  // extension of this build: variadic (value, index) reduce -> argmax
  TOP_ARGMAX_SEG = 19,
  TOP_GEMV = 20,
  TOP_DECODE_ATTN = 21,
  TOP_COUNT = 22
};

// ---- elementwise subops (vm_common.cl:118-146) -----------------------------------
enum EwSub : uint32_t {
  SUB_ADD = 0, SUB_MUL, SUB_SUB, SUB_DIV, SUB_MAX, SUB_MIN, SUB_POW,
  SUB_COPY, SUB_NEG, SUB_EXP, SUB_LOG, SUB_SQRT, SUB_RSQRT, SUB_TANH,
  SUB_ABS, SUB_FLOOR, SUB_CEIL, SUB_SIGN, SUB_FILL, SUB_IOTA_FLAT,
  SUB_CMP, SUB_SELECT, SUB_LTS, SUB_CONVERT, SUB_BITCAST,
  SUB_ATAN2, SUB_REMAINDER,
  SUB_LOG1P, SUB_EXPM1, SUB_CBRT, SUB_SIN, SUB_COS, SUB_TAN,
  SUB_RINT, SUB_ROUND,
  SUB_AND, SUB_OR, SUB_XOR, SUB_NOT,
  SUB_ISFINITE, SUB_AFFINE, SUB_GELU,
  SUB_SHL, SUB_SHR_L, SUB_SHR_A,
  SUB_COUNT
};

// LAYERNORM_SEG p3 flags (extension; 0 = the reference's one-pass core op)
enum : uint32_t { LN_AFFINE = 1, LN_GELU = 2, LN_TWO_PASS = 4 };

// ---- entry sentinels (scheduler.py:80-85) -----------------------------------------
constexpr uint32_t ENT_NOP = 0xFFFFFFFFu;
constexpr uint32_t ENT_BARRIER = 0xFFFFFFFEu;
constexpr uint32_t ENT_WHILE = 0xFFFFFFFDu;
constexpr uint32_t ENT_IF = 0xFFFFFFFCu;
constexpr uint32_t ENT_FOR = 0xFFFFFFFBu;
constexpr uint32_t FLAG_NONE = 0xFFFFFFFFu;

// A buffer handle is an arena byte offset, or a port index with bit 31 set
// (vm_common.cl:41-45).  Ports are caller-owned device buffers bound per execute.
constexpr uint32_t PORT_BIT = 0x80000000u;

// TOP_DECODE_ATTN: key splits per head at most, cache keys per split at most.
constexpr uint32_t kDecMaxSplits = 1024;
constexpr uint32_t kDecSplitKeys = 64;
// TOP_ARGMAX_SEG: splits per row at most.
constexpr uint32_t kArgmaxMaxSplits = 256;
// TOP_GEMV: rows (M) per task at most.
constexpr uint32_t kGemvMaxM = 8;
// TOP_MMA: log2 of the K split (task p3 bits 28-31) at most.
constexpr uint32_t kMmaMaxSplitLog2 = 5;
constexpr int kMaxPorts = 256;          // power of two: handles mask the port index

// Per-program control buffer: status words, then one arrival word per lane.
constexpr uint32_t kMaxLanes = 4096;
enum : uint32_t {
  BAR_GEN = 1,        // release epoch, written by lane 0 when every lane arrived
  BAR_ERROR = 2,      // nonzero: a lane aborted (see VmError)
  BAR_ERRINFO = 3,    // lane / detail of the first error
  BAR_FLAGS = 64,     // [kMaxLanes] arrival epochs, one word per lane
  BAR_XGEN = BAR_FLAGS + kMaxLanes,   // [kXcds] copies of the release epoch, one cache line apart
  BAR_WORDS = BAR_XGEN + 8 * 32
};
// XCDs per device: workgroup i of a launch is dispatched to XCD i % kXcds.
constexpr uint32_t kXcds = 8;
// Profiling counters (100 MHz ticks of s_memrealtime): [0] lane-time in grid
// barriers, [1] lane-barriers, [2] lane-time from launch start to the lane's
// end, [3] lane-time waiting for completion flags; task i at kStatTask + 4 i:
// lane-time summed over its entries, longest single entry, entry count.
constexpr uint32_t kStatTask = 4;

enum VmError : uint32_t {
  VM_OK = 0,
  VM_ERR_BARRIER_TIMEOUT = 1,
  VM_ERR_FRAME_DEPTH = 2,
  VM_ERR_BAD_ENTRY = 3,
  VM_ERR_BAD_TASK = 4,
};

struct Task {          // 48 bytes, scheduler.py:100
  uint32_t tile_op;    // op | dtype << 8 | adtype << 16
  uint32_t dst, a, b;
  uint32_t p[8];
};
static_assert(sizeof(Task) == 48, "Task layout");

struct Entry {         // 32 bytes, scheduler.py:102
  uint32_t task, tile_lo, tile_hi, wait_flag, wait_count, signal_flag, slots, pad;
};
static_assert(sizeof(Entry) == 32, "Entry layout");

struct LaneSpan {      // 16 bytes, scheduler.py:101
  uint32_t off, count, root_len, pad;
};
static_assert(sizeof(LaneSpan) == 16, "LaneSpan layout");

// Kernel arguments of the persistent VM (passed by value in the kernarg segment).
struct VmArgs {
  uint8_t* arena;
  const int32_t* aux;
  const Task* tasks;
  const Entry* entries;
  const LaneSpan* lanes;
  uint32_t* ctl;            // BAR_WORDS control words (status + arrival flags)
  uint32_t n_lanes;
  uint32_t ew_ts;           // elements per EW tile (scheduler PJRT_OCL_EW_TS)
  uint32_t mma_t;           // default MMA output tile edge (PJRT_OCL_MMA_T)
  uint32_t timeout_ticks;   // barrier wait limit in s_memrealtime ticks (100 MHz)
  uint64_t* stats;          // profiling counters (null: off), see kStat*
  uint8_t* scratch;         // loader-owned scratch, zeroed at load (split partials, arrival counters)
  const uint32_t* task_scratch;   // per task: byte offset of its scratch region
  uint64_t* flags;          // completion flags (extension), n_flags words in the scratch; null: none
  uint32_t seq;             // this launch's sequence number (the high half of a flag value)
  uint32_t pad_;
  uint8_t* ports[kMaxPorts];
};

}  // namespace vm

// FeLLM kernel-plugin C ABI for the gfx950 kernels.
//
// Mirrors what plugins/cuda_kernels/src/lib.rs and launchers.rs export to
// fellm-plugin-host (crates/fellm-plugin-host/src/loader.rs:363-437,
// registry.rs): ABI version 0.9.0, a JSON manifest, init with a HostContext,
// per-op registration under (op, input dtypes, output dtype) keys, and
// launchers with the PluginLaunchFn signature.
//
// Buffer contract (plugins/cuda_kernels/src/buffers.rs:119-560,
// launchers.rs:147-189): TensorRef/TensorMut data are HOST pointers owned by
// the caller.  The plugin keeps a device mirror per (host ptr, byte length):
//   * immutable weights (logical_id != 0) are uploaded once per logical id;
//   * activations are uploaded unless the mirror is already device-valid;
//   * outputs are produced on the device and marked device-valid; they are
//     copied back only when FELLM_ROCM_SYNC_OUTPUTS (or the reference's
//     FELLM_CUDA_SYNC_OUTPUTS) is set, or by an explicit Cast launch;
//   * _fellm_plugin_invalidate_f32 marks a mirror stale after a host write;
//   * _fellm_plugin_register_device_tensor binds a host view to an existing
//     device allocation (no copies at all).
// All work runs on one non-blocking stream of default priority, exported by
// _fellm_plugin_device_stream.  Launches are serialised by a process mutex,
// as in the reference.  Every entry point catches exceptions (-99).
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "fellm_abi.h"
#include "fellm_rocm.h"

namespace {

// ---------------------------------------------------------------------------
// Custom op ids: OpKind::custom(ns, name) (crates/fellm-plugin-abi/src/op.rs:69-80).
// ---------------------------------------------------------------------------
constexpr uint32_t custom_op(const char *ns, const char *name) {
    uint32_t h = 0x811c9dc5u;
    for (const char *p = ns; *p; ++p) h = (h ^ (uint8_t)*p) * 0x01000193u;
    h = (h ^ (uint8_t)':') * 0x01000193u;
    for (const char *p = name; *p; ++p) h = (h ^ (uint8_t)*p) * 0x01000193u;
    return h | FELLM_OP_CUSTOM_TAG;
}
constexpr uint32_t kOpAddRmsNorm = custom_op("rocm", "add_rmsnorm");
constexpr uint32_t kOpRopeKvWrite = custom_op("rocm", "rope_kv_write");
constexpr uint32_t kOpRouterTopK = custom_op("rocm", "router_topk");
constexpr uint32_t kOpEmbeddingRmsNorm = custom_op("rocm", "embedding_rmsnorm");

struct LaunchError {
    int code;
};
[[noreturn]] void fail(int code) { throw LaunchError{code}; }
void check(int rc) {
    if (rc != 0) fail(rc);
}
void hip_check(hipError_t e, int code = FELLM_ERR_ALLOC) {
    if (e != hipSuccess) fail(code);
}

// ---------------------------------------------------------------------------
// Process state.
// ---------------------------------------------------------------------------
struct Mirror {
    void *dev = nullptr;
    size_t bytes = 0;
    bool device_valid = false;
    // While !device_valid: bytes [0, valid_prefix) of the device copy already
    // equal the host's (an input read row by row, such as a K/V buffer that
    // grows by one row per decode step, uploads only the rows it lacks).
    size_t valid_prefix = 0;
};

struct State {
    std::mutex mu;
    bool have_ctx = false;
    FellmHostContext ctx{};
    hipStream_t stream = nullptr;
    std::map<std::pair<uintptr_t, size_t>, Mirror> act;          // activations
    std::unordered_map<uint64_t, Mirror> weights;                 // logical_id (or ptr) -> mirror
    std::map<std::pair<uintptr_t, size_t>, uint64_t> external;   // registered device tensors
    Mirror step_params;                                          // DeviceStepParams block
    bool step_valid = false;                                     // step_params has been written
    Mirror step_kv_pos;                                          // u32: the single row's KV position
    bool capturing = false;                                      // stream is being captured (this launch)
    Mirror scratch;                                              // per-launch small uploads
    Mirror attn_ws;                                              // split-key attention partial sums
    void *pinned = nullptr;                                      // host staging for `scratch`
    size_t pinned_bytes = 0;
    bool host_reads_pending = false;  // an H2D copy may still read caller memory
    int sync_outputs = -1;
    // Output mirrors this launch marked stale, with their previous state, so
    // that a launch failing before its kernel runs leaves them as they were.
    std::vector<std::pair<Mirror *, bool>> touched_outputs;
};

State &state() {
    static State *s = new State();  // never destroyed: device memory outlives static teardown
    return *s;
}

hipStream_t stream_locked(State &st) {
    if (!st.stream) hip_check(hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking));
    return st.stream;
}

// Whether the plugin stream is being captured.  A stream that does not exist
// yet cannot be (captures start on the stream _fellm_plugin_device_stream
// hands out), and asking must not create one: error paths that need no GPU
// stay GPU-free.
bool stream_capturing(State &st) {
    if (!st.stream) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st.stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusActive;
}

bool sync_outputs(State &st) {
    if (st.sync_outputs < 0) {
        auto on = [](const char *name) {
            const char *v = std::getenv(name);
            return v && std::strcmp(v, "0") != 0 && std::strcmp(v, "false") != 0 && std::strcmp(v, "off") != 0;
        };
        st.sync_outputs = (on("FELLM_ROCM_SYNC_OUTPUTS") || on("FELLM_CUDA_SYNC_OUTPUTS")) ? 1 : 0;
    }
    return st.sync_outputs == 1;
}

State &state();

// Allocations, uploads, staging and host reads cannot be recorded into a
// graph: a launch captured into one must find every buffer already resident
// (a warm-up launch outside the capture does that) and reads its per-step
// values from the DeviceStepParams block.
void no_capture() {
    if (state().capturing) fail(FELLM_ERR_LAUNCH);
}

void ensure_capacity(Mirror &m, size_t bytes) {
    if (m.dev && m.bytes >= bytes) return;
    no_capture();
    if (m.dev) hip_check(hipFree(m.dev));
    m.dev = nullptr;
    m.bytes = 0;
    m.device_valid = false;
    m.valid_prefix = 0;
    hip_check(hipMalloc(&m.dev, bytes ? bytes : 1));
    m.bytes = bytes;
}

// H2D copy from caller-owned memory.  The caller owns its buffers only for
// the duration of the launch, so a launch that uploaded anything waits for
// its stream before returning (see guarded()).
void upload(State &st, void *dev, const void *host, size_t bytes) {
    if (!bytes) return;
    no_capture();
    hip_check(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, stream_locked(st)));
    st.host_reads_pending = true;
}

const uint64_t *find_external(State &st, const void *host, size_t bytes) {
    auto it = st.external.find({reinterpret_cast<uintptr_t>(host), bytes});
    return it == st.external.end() ? nullptr : &it->second;
}

// Device address of an input, uploading it if needed.
void *ensure_input(State &st, const FellmTensorRef &t) {
    if (!t.data || t.byte_len == 0) fail(FELLM_ERR_ARITY);
    if (const uint64_t *ext = find_external(st, t.data, t.byte_len)) return reinterpret_cast<void *>(*ext);
    if (t.logical_id != 0) {
        Mirror &m = st.weights[t.logical_id];
        if (!m.device_valid || m.bytes != t.byte_len) {
            ensure_capacity(m, t.byte_len);
            m.bytes = t.byte_len;
            upload(st, m.dev, t.data, t.byte_len);
            m.device_valid = true;
        }
        return m.dev;
    }
    Mirror &m = st.act[{reinterpret_cast<uintptr_t>(t.data), (size_t)t.byte_len}];
    if (!m.device_valid) {
        ensure_capacity(m, t.byte_len);
        upload(st, static_cast<uint8_t *>(m.dev) + m.valid_prefix, static_cast<const uint8_t *>(t.data) + m.valid_prefix,
               t.byte_len - m.valid_prefix);
        m.device_valid = true;
        m.valid_prefix = 0;
    }
    return m.dev;
}

// Device address of an activation input of which a launch reads only the
// first `bytes`: the mirror is keyed by the whole tensor (as every other
// launch keys it) and only the rows it does not hold yet are uploaded.
void *ensure_input_prefix(State &st, const FellmTensorRef &t, size_t bytes) {
    if (!t.data || t.byte_len == 0) fail(FELLM_ERR_ARITY);
    if (bytes >= t.byte_len || t.logical_id != 0 || find_external(st, t.data, t.byte_len)) return ensure_input(st, t);
    Mirror &m = st.act[{reinterpret_cast<uintptr_t>(t.data), (size_t)t.byte_len}];
    if (m.device_valid) return m.dev;
    ensure_capacity(m, t.byte_len);
    if (m.valid_prefix < bytes) {
        upload(st, static_cast<uint8_t *>(m.dev) + m.valid_prefix, static_cast<const uint8_t *>(t.data) + m.valid_prefix,
               bytes - m.valid_prefix);
        m.valid_prefix = bytes;
    }
    return m.dev;
}

// Device address of an output mirror (no upload unless `inout`).
void *ensure_output(State &st, const FellmTensorMut &t, bool inout = false) {
    if (!t.data || t.byte_len == 0) fail(FELLM_ERR_ARITY);
    if (const uint64_t *ext = find_external(st, t.data, t.byte_len)) return reinterpret_cast<void *>(*ext);
    Mirror &m = st.act[{reinterpret_cast<uintptr_t>(t.data), (size_t)t.byte_len}];
    if (!m.dev || m.bytes < t.byte_len) {
        const bool had = m.device_valid && m.dev;
        if (had) fail(FELLM_ERR_SHAPE);
        ensure_capacity(m, t.byte_len);
    }
    if (inout && !m.device_valid) upload(st, m.dev, t.data, t.byte_len);
    st.touched_outputs.emplace_back(&m, m.device_valid);
    m.device_valid = false;  // until the launch completes on the stream
    m.valid_prefix = 0;      // the device copy no longer follows the host's
    return m.dev;
}

// Marks outputs device-valid and downloads them when sync is requested
// (launchers.rs:174-189).
void finish_outputs(State &st, FellmTensorMut *outs, uint32_t n, bool sync_host = false) {
    const bool sync = !st.capturing && (sync_host || sync_outputs(st));
    for (uint32_t i = 0; i < n; ++i) {
        if (!outs[i].data) continue;
        if (find_external(st, outs[i].data, outs[i].byte_len)) continue;
        auto it = st.act.find({reinterpret_cast<uintptr_t>(outs[i].data), (size_t)outs[i].byte_len});
        if (it == st.act.end()) continue;
        it->second.device_valid = true;
        if (sync)
            hip_check(hipMemcpyAsync(outs[i].data, it->second.dev, outs[i].byte_len, hipMemcpyDeviceToHost,
                                     stream_locked(st)));
    }
    if (sync) hip_check(hipStreamSynchronize(stream_locked(st)));
}

// Small per-launch host arrays (positions, block tables, ids) staged through
// one growing device buffer.  The copy is ordered on the plugin stream before
// the kernel that reads it; the host waits for the stream before reusing it.
void *stage_small(State &st, const std::vector<const void *> &srcs, const std::vector<size_t> &sizes,
                  std::vector<void *> &dsts) {
    no_capture();
    size_t total = 0;
    std::vector<size_t> offs;
    for (size_t sz : sizes) {
        offs.push_back(total);
        total += (sz + 255) / 256 * 256;
    }
    hip_check(hipStreamSynchronize(stream_locked(st)));  // earlier readers of scratch/pinned are done
    ensure_capacity(st.scratch, total);
    if (st.pinned_bytes < total) {
        if (st.pinned) hip_check(hipHostFree(st.pinned));
        st.pinned = nullptr;
        st.pinned_bytes = 0;
        hip_check(hipHostMalloc(&st.pinned, total, hipHostMallocDefault));
        st.pinned_bytes = total;
    }
    dsts.clear();
    for (size_t i = 0; i < srcs.size(); ++i) {
        std::memcpy(static_cast<uint8_t *>(st.pinned) + offs[i], srcs[i], sizes[i]);
        dsts.push_back(static_cast<uint8_t *>(st.scratch.dev) + offs[i]);
    }
    hip_check(hipMemcpyAsync(st.scratch.dev, st.pinned, total, hipMemcpyHostToDevice, stream_locked(st)));
    return st.scratch.dev;
}

bool snapshot(State &st, FellmPagedKvSnapshot &out) {
    if (!st.have_ctx || !st.ctx.snapshot_paged) return false;
    std::memset(&out, 0, sizeof(out));
    return st.ctx.snapshot_paged(&out) == 0;
}

size_t dtype_size(uint32_t dt) {
    switch (dt) {
        case FELLM_DTYPE_F32:
        case FELLM_DTYPE_U32:
        case FELLM_DTYPE_I32: return 4;
        case FELLM_DTYPE_F16:
        case FELLM_DTYPE_BF16: return 2;
        default: return 0;
    }
}

size_t elems(const FellmTensorRef &t, uint32_t dt) {
    const size_t es = dtype_size(dt);
    if (!es || t.byte_len % es) fail(FELLM_ERR_SHAPE);
    return t.byte_len / es;
}
size_t elems(const FellmTensorMut &t, uint32_t dt) {
    const size_t es = dtype_size(dt);
    if (!es || t.byte_len % es) fail(FELLM_ERR_SHAPE);
    return t.byte_len / es;
}

template <typename Body>
int guarded(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
            uint32_t n_out, uint32_t min_in, uint32_t min_out, bool need_attrs, Body &&body) {
    try {
        if (!in || !out || n_in < min_in || n_out < min_out || (need_attrs && !attrs)) return FELLM_ERR_ARITY;
        State &st = state();
        std::lock_guard<std::mutex> lock(st.mu);
        st.host_reads_pending = false;
        st.capturing = stream_capturing(st);
        st.touched_outputs.clear();
        try {
            body(st);
        } catch (const LaunchError &e) {
            // A rejected launch (argument, shape or dtype checks, which run
            // before anything is enqueued) restores its outputs' mirror state:
            // a mirror holding device-only data must not fall back to the
            // caller's stale host bytes.  After a failed kernel launch the
            // device copy may be partly written, so it stays stale.
            if (e.code != FELLM_ERR_LAUNCH)
                for (auto it = st.touched_outputs.rbegin(); it != st.touched_outputs.rend(); ++it)
                    it->first->device_valid = it->second;
            st.touched_outputs.clear();
            throw;
        }
        st.touched_outputs.clear();
        if (st.host_reads_pending) {
            st.host_reads_pending = false;
            hip_check(hipStreamSynchronize(stream_locked(st)));
        }
        return FELLM_OK;
    } catch (const LaunchError &e) {
        return e.code;
    } catch (...) {
        return FELLM_ERR_PANIC;
    }
}

void *stream_ptr(State &st) { return reinterpret_cast<void *>(stream_locked(st)); }

// Device address of a u32 field of the DeviceStepParams block (word index:
// 0 token_id, 1 position, 2 sequence_length, 5 kv_write_slot), or NULL before
// the first _fellm_plugin_update_step_params.  Single-row decode launches read
// these instead of host values, as the CUDA plugin's controlled kernels do, so
// that a captured step replays with the values of the step being replayed.
const uint32_t *step_u32(State &st, size_t word) {
    if (!st.step_valid || !st.step_params.dev) return nullptr;
    return static_cast<const uint32_t *>(st.step_params.dev) + word;
}

// The single row's KV position from the step block (device-side; see
// fellm_rocm_step_kv_position), or NULL without a step block.
const uint32_t *step_kv_position(State &st, uint32_t block_size) {
    if (!st.step_valid || !st.step_params.dev) return nullptr;
    ensure_capacity(st.step_kv_pos, 4);
    check(fellm_rocm_step_kv_position(static_cast<const FellmDeviceStepParams *>(st.step_params.dev), block_size,
                                      static_cast<uint32_t *>(st.step_kv_pos.dev), stream_ptr(st)));
    return static_cast<const uint32_t *>(st.step_kv_pos.dev);
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------

// RmsNorm [x, w] -> y.  Groups of w.len() (backend.rs:1104-1133 and
// launchers.rs:336-401 both reduce to this when x.len() % w.len() == 0).
int launch_rmsnorm(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                   uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 2, 1, true, [&](State &st) {
        const uint32_t dt = in[0].dtype;
        if (in[1].dtype != FELLM_DTYPE_F32 || out[0].dtype != dt) fail(FELLM_ERR_DTYPE);
        const size_t n = elems(in[0], dt), g = elems(in[1], FELLM_DTYPE_F32);
        if (elems(out[0], dt) != n || g == 0 || n % g) fail(FELLM_ERR_SHAPE);
        void *x = ensure_input(st, in[0]);
        void *w = ensure_input(st, in[1]);
        void *y = ensure_output(st, out[0]);
        check(fellm_rocm_add_rmsnorm(x, nullptr, nullptr, dt, (const float *)w, (uint32_t)g, y, dt, n, attrs->eps,
                                     stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

// Custom rocm:add_rmsnorm [x, residual, w] -> [h, y].
int launch_add_rmsnorm(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                       uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 3, 2, true, [&](State &st) {
        const uint32_t dt = in[0].dtype;
        if (in[1].dtype != dt || in[2].dtype != FELLM_DTYPE_F32 || out[0].dtype != dt || out[1].dtype != dt)
            fail(FELLM_ERR_DTYPE);
        const size_t n = elems(in[0], dt), g = elems(in[2], FELLM_DTYPE_F32);
        if (elems(in[1], dt) != n || elems(out[0], dt) != n || elems(out[1], dt) != n || g == 0 || n % g)
            fail(FELLM_ERR_SHAPE);
        void *x = ensure_input(st, in[0]);
        void *r = ensure_input(st, in[1]);
        void *w = ensure_input(st, in[2]);
        void *h = ensure_output(st, out[0]);
        void *y = ensure_output(st, out[1]);
        check(fellm_rocm_add_rmsnorm(x, r, h, dt, (const float *)w, (uint32_t)g, y, dt, n, attrs->eps, stream_ptr(st)));
        finish_outputs(st, out, 2);
    });
}

// Add [a, b] -> out (backend.rs:1543-1553).
int launch_add(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
               uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 2, 1, false, [&](State &st) {
        const uint32_t dt = in[0].dtype;
        if (in[1].dtype != dt || out[0].dtype != dt) fail(FELLM_ERR_DTYPE);
        const size_t n = elems(in[0], dt);
        if (elems(in[1], dt) != n || elems(out[0], dt) != n) fail(FELLM_ERR_SHAPE);
        void *a = ensure_input(st, in[0]);
        void *b = ensure_input(st, in[1]);
        void *o = ensure_output(st, out[0]);
        check(fellm_rocm_add(a, b, dt, o, dt, n, stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

// SiluGate [gate, up] -> out (backend.rs:1174-1184, launchers.rs:192-234).
int launch_silu_gate(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                     uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 2, 1, false, [&](State &st) {
        const uint32_t dt = in[0].dtype;
        if (in[1].dtype != dt || out[0].dtype != dt) fail(FELLM_ERR_DTYPE);
        const size_t n = elems(in[0], dt);
        if (elems(in[1], dt) != n || elems(out[0], dt) != n) fail(FELLM_ERR_SHAPE);
        void *g = ensure_input(st, in[0]);
        void *u = ensure_input(st, in[1]);
        void *o = ensure_output(st, out[0]);
        check(fellm_rocm_silu_gate(g, u, dt, o, dt, n, stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

// Per-row RoPE positions, as backend.rs:1148-1151: the paged context's
// row_rope_positions[row] when present, else attrs.position + row.
std::vector<uint32_t> rope_positions(State &st, const FellmOpAttrs &a, uint32_t rows, bool &any) {
    std::vector<uint32_t> pos(rows);
    FellmPagedKvSnapshot snap;
    any = false;
    const bool have = snapshot(st, snap) && snap.row_rope_positions;
    for (uint32_t r = 0; r < rows; ++r) {
        if (have && r < snap.batch_size) {
            pos[r] = snap.row_rope_positions[r];
            any = true;
        } else {
            const uint64_t p = (uint64_t)a.position + r;
            pos[r] = p > 0xffffffffull ? 0xffffffffu : (uint32_t)p;  // saturating_add
        }
    }
    return pos;
}

// Rope [x, inv_freqs] -> out (backend.rs:1135-1172).
int launch_rope(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 2, 1, true, [&](State &st) {
        const FellmOpAttrs &a = *attrs;
        const uint32_t dt = in[0].dtype;
        if (in[1].dtype != FELLM_DTYPE_F32 || out[0].dtype != dt) fail(FELLM_ERR_DTYPE);
        // custom_op_id 1 asks backend-cpu to copy the pre-rotation rows into
        // the process's pre-RoPE key store (backend.rs:1152-1158).  Across the
        // plugin C ABI there is no channel to that store (HostContext carries
        // none; the CUDA plugin's call, launchers.rs:430-444, reaches its own
        // never-installed copy of the store, c_abi.rs:40-44), so, like the
        // CUDA plugin, the launch rotates and leaves the store alone.
        const size_t n = elems(in[0], dt);
        if (elems(out[0], dt) != n) fail(FELLM_ERR_SHAPE);
        const size_t nh = a.n_heads ? a.n_heads : 1, hd = a.head_dim ? a.head_dim : 1;
        const size_t width = nh * hd;
        if (n % width || elems(in[1], FELLM_DTYPE_F32) < a.rope_dim / 2) fail(FELLM_ERR_SHAPE);
        const uint32_t rows = (uint32_t)(n / width);
        bool any = false;
        std::vector<uint32_t> pos = rope_positions(st, a, rows, any);
        void *x = ensure_input(st, in[0]);
        void *f = ensure_input(st, in[1]);
        void *o = ensure_output(st, out[0]);
        std::vector<void *> d;
        // A decode row takes its position from the step block when there is
        // one (rope_controlled: launchers.rs:479-497, used unless the
        // snapshot holds a batch of more than one row).
        const uint32_t *pd = rows == 1 ? step_u32(st, 1) : nullptr;
        if (!pd && any) {
            stage_small(st, {pos.data()}, {pos.size() * 4}, d);
            pd = static_cast<const uint32_t *>(d[0]);
        }
        check(fellm_rocm_rope(x, o, (uint32_t)nh, nullptr, nullptr, 0, dt, rows, (uint32_t)hd, a.rope_dim,
                              a.rope_pairing, (const float *)f, pd, a.position, stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

// Paged geometry from the host snapshot (paged_ctx.rs:14-53); the arena must
// be device-resident (the ROCm backend allocates it in HBM).  The block table
// is the snapshot's device-resident table when it holds at least the host
// table's entries (then its logical stride applies: launchers.rs:3963-3985),
// else the host table staged for this launch.  pos_a / pos_b (may be NULL)
// are staged too, n_pos entries each (0: the snapshot's batch size); their
// device addresses come back in dev_a / dev_b.
FellmRocmPagedKv paged_geometry(State &st, const FellmPagedKvSnapshot &snap, uint32_t layer, uint32_t kv_dtype,
                                const uint32_t *pos_a, const uint32_t **dev_a, const uint32_t *pos_b = nullptr,
                                const uint32_t **dev_b = nullptr, size_t n_pos = 0) {
    const size_t npos = n_pos ? n_pos : snap.batch_size;
    if (!snap.device_arena || snap.device_arena_len == 0) fail(FELLM_ERR_PAGED_NO_DEVICE);
    if (snap.elem_bytes != 2 || !snap.block_table || snap.block_size == 0 || snap.tokens_stride == 0)
        fail(FELLM_ERR_PAGED_RANGE);
    const bool device_table = snap.device_block_table && snap.n_device_block_table >= snap.n_block_table &&
                              snap.device_logical_stride > 0;
    std::vector<const void *> srcs;
    std::vector<size_t> sizes;
    if (!device_table) {
        srcs.push_back(snap.block_table);
        sizes.push_back(snap.n_block_table * 4);
    }
    if (pos_a) {
        srcs.push_back(pos_a);
        sizes.push_back(npos * 4);
    }
    if (pos_b) {
        srcs.push_back(pos_b);
        sizes.push_back(npos * 4);
    }
    std::vector<void *> staged;
    if (!srcs.empty()) stage_small(st, srcs, sizes, staged);
    size_t i = 0;
    FellmRocmPagedKv kv{};
    kv.arena = snap.device_arena;
    kv.arena_len = snap.device_arena_len;
    if (device_table) {
        kv.block_table = snap.device_block_table;
        kv.n_block_table = snap.n_device_block_table;
        kv.n_logical_blocks = (uint32_t)snap.device_logical_stride;
    } else {
        kv.block_table = static_cast<const uint32_t *>(staged[i++]);
        kv.n_block_table = snap.n_block_table;
        kv.n_logical_blocks = (uint32_t)snap.n_logical_blocks;
    }
    if (pos_a && dev_a) *dev_a = static_cast<const uint32_t *>(staged[i]);
    if (pos_a) ++i;
    if (pos_b && dev_b) *dev_b = static_cast<const uint32_t *>(staged[i]);
    kv.n_layers = (uint32_t)snap.n_layers;
    kv.layer = layer;
    kv.block_size = (uint32_t)snap.block_size;
    kv.block_bytes = snap.block_bytes;
    kv.stride = (uint32_t)snap.tokens_stride;
    kv.kv_dtype = kv_dtype;
    return kv;
}

// Host-side check of every batch row's K/V slot against the snapshot, as the
// CUDA plugin does before launching (launchers.rs:3913-3945): the table must
// hold the layer, the logical block must exist, and the slot's block must lie
// inside the device arena.  The kernels then run without an error word, so
// no launch waits for a device-to-host read.
void check_slots(const FellmPagedKvSnapshot &snap, uint32_t layer, const uint32_t *positions, size_t batch) {
    const size_t n_logical = snap.n_logical_blocks;
    if (!n_logical || !snap.block_bytes || !snap.block_size || layer >= snap.n_layers) fail(FELLM_ERR_PAGED_RANGE);
    const uint64_t row_bytes = (uint64_t)snap.tokens_stride * 2;
    for (size_t b = 0; b < batch; ++b) {
        const uint64_t pos = positions[b];
        const uint64_t logical = pos / snap.block_size, slot = pos % snap.block_size;
        if (logical >= n_logical) fail(FELLM_ERR_PAGED_RANGE);
        const uint64_t idx = ((uint64_t)b * snap.n_layers + layer) * n_logical + logical;
        if (idx >= snap.n_block_table) fail(FELLM_ERR_PAGED_RANGE);
        const uint64_t base = (uint64_t)snap.block_table[idx] * snap.block_bytes + slot * row_bytes;
        if (base + (uint64_t)snap.block_size * row_bytes + row_bytes > snap.device_arena_len) fail(FELLM_ERR_PAGED_RANGE);
    }
}

// KvWrite [row(s), (cache)] -> cache (backend.rs:1734-1793, launchers.rs:3770-3900).
int launch_kv_write(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                    uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 1, 1, true, [&](State &st) {
        const FellmOpAttrs &a = *attrs;
        const uint32_t dt = in[0].dtype;
        if (dt != FELLM_DTYPE_F32 && dt != FELLM_DTYPE_F16 && dt != FELLM_DTYPE_BF16) fail(FELLM_ERR_DTYPE);
        const size_t n = elems(in[0], dt);
        FellmPagedKvSnapshot snap;
        const bool paged = a.block_size > 0 && snapshot(st, snap);
        if (paged) {
            const size_t batch = snap.batch_size ? snap.batch_size : 1;
            if (snap.tokens_stride == 0 || n != batch * snap.tokens_stride) fail(FELLM_ERR_SHAPE);
            void *rows = ensure_input(st, in[0]);
            // A single row takes its slot from the step block when there is
            // one (kv_write_row, launchers.rs:3993-4010), else the snapshot.
            const bool controlled = batch == 1 && step_u32(st, 2);
            if (!controlled && !snap.row_positions) fail(FELLM_ERR_PAGED_MISSING);
            const uint32_t *pos = nullptr;
            FellmRocmPagedKv kv = paged_geometry(st, snap, a.layer_ord, FELLM_DTYPE_F16,
                                                 controlled ? nullptr : snap.row_positions, &pos);
            if (controlled)
                pos = step_kv_position(st, kv.block_size);  // device-side slot: out-of-range rows are skipped
            else
                check_slots(snap, a.layer_ord, snap.row_positions, batch);
            check(fellm_rocm_kv_write(rows, dt, (uint32_t)batch, pos, &kv, a.kv_slot != 0, nullptr, stream_ptr(st)));
            finish_outputs(st, out, 0);
            return;
        }
        // Contiguous layout (also when block_size > 0 but no paged context is
        // installed, as backend.rs:1742 does): kv_buf [max_seq, dim] of the
        // row dtype, row written at attrs.position.
        FellmTensorMut &buf = out[0];
        if (buf.dtype != dt || buf.rank != 2) fail(FELLM_ERR_SHAPE);
        const size_t max_seq = buf.dims[0], dim = buf.dims[1];
        if (n != dim) fail(FELLM_ERR_SHAPE);
        if (a.position >= max_seq) fail(FELLM_ERR_SHAPE);
        if (elems(buf, dt) < max_seq * dim) fail(FELLM_ERR_SHAPE);
        void *row = ensure_input(st, in[0]);
        void *cache = ensure_output(st, buf, /*inout=*/true);
        const size_t es = dtype_size(dt);
        hip_check(hipMemcpyAsync(static_cast<uint8_t *>(cache) + (size_t)a.position * dim * es, row, dim * es,
                                 hipMemcpyDeviceToDevice, stream_locked(st)),
                  FELLM_ERR_LAUNCH);
        finish_outputs(st, out, 1);
    });
}

// Custom rocm:rope_kv_write [q, k, v, inv_freqs] -> [q_out, (k_out)].
// attrs: n_heads, n_kv_heads, head_dim, rope_dim, rope_pairing, layer_ord,
// cast_to = cache dtype (BF16, else F16 as in the reference arena).
int launch_rope_kv_write(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                         uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 4, 1, true, [&](State &st) {
        const FellmOpAttrs &a = *attrs;
        const uint32_t dt = in[0].dtype;
        if (in[1].dtype != dt || in[2].dtype != dt || in[3].dtype != FELLM_DTYPE_F32 || out[0].dtype != dt)
            fail(FELLM_ERR_DTYPE);
        FellmPagedKvSnapshot snap;
        if (!snapshot(st, snap)) fail(FELLM_ERR_PAGED_MISSING);
        const size_t batch = snap.batch_size ? snap.batch_size : 1;
        // One decode row: RoPE position and KV slot from the step block.
        const bool controlled = batch == 1 && step_u32(st, 2);
        if (!controlled && !snap.row_positions) fail(FELLM_ERR_PAGED_MISSING);
        const size_t hd = a.head_dim, nq = a.n_heads, nkv = a.n_kv_heads;
        if (!hd || !nq || !nkv) fail(FELLM_ERR_SHAPE);
        if (elems(in[0], dt) != batch * nq * hd || elems(in[1], dt) != batch * nkv * hd ||
            elems(in[2], dt) != batch * nkv * hd || elems(out[0], dt) != batch * nq * hd ||
            snap.tokens_stride != nkv * hd)
            fail(FELLM_ERR_SHAPE);
        const bool has_kout = n_out >= 2 && out[1].data;
        if (has_kout && (out[1].dtype != dt || elems(out[1], dt) != batch * nkv * hd)) fail(FELLM_ERR_SHAPE);
        void *q = ensure_input(st, in[0]);
        void *k = ensure_input(st, in[1]);
        void *v = ensure_input(st, in[2]);
        void *f = ensure_input(st, in[3]);
        void *qo = ensure_output(st, out[0]);
        void *ko = has_kout ? ensure_output(st, out[1]) : nullptr;
        const uint32_t kv_dt = a.cast_to == FELLM_DTYPE_BF16 ? FELLM_DTYPE_BF16 : FELLM_DTYPE_F16;
        const uint32_t *kv_pos = nullptr, *rope_pos = nullptr;
        FellmRocmPagedKv kv;
        if (controlled) {
            kv = paged_geometry(st, snap, a.layer_ord, kv_dt, nullptr, nullptr);
            kv_pos = step_kv_position(st, kv.block_size);
            rope_pos = step_u32(st, 1);
        } else {
            kv = paged_geometry(st, snap, a.layer_ord, kv_dt, snap.row_positions, &kv_pos, snap.row_rope_positions,
                                &rope_pos);
        }
        if (!controlled) check_slots(snap, a.layer_ord, snap.row_positions, batch);
        check(fellm_rocm_rope_kv_write(q, qo, (uint32_t)nq, k, ko, v, (uint32_t)nkv, dt, (uint32_t)batch, (uint32_t)hd,
                                       a.rope_dim, a.rope_pairing, (const float *)f, rope_pos, kv_pos, &kv, nullptr,
                                       stream_ptr(st)));
        finish_outputs(st, out, has_kout ? 2 : 1);
    });
}

// Attention [q, k, v] -> out in its paged decode form (block_size > 0 with a
// paged context): backend.rs:1244-1368 and the CUDA plugin's paged decode
// paths (launchers.rs:3243-3560).  A physical batch (batch_size > 1 or q wider
// than one row) attends row r to row_lengths[r] keys, causal with
// attention_window; a single sequence attends to past_len + 1 keys, causal
// when attention_mode == 0.  K/V come from the device arena (f16, or bf16 when
// cast_to is BF16, as rope_kv_write writes it).  block_size == 0 and the canvas
// form go to launch_attention_f32kv.
// The non-paged Attention arms, f32 throughout (as both reference backends
// read these K/V inputs as f32):
//  * contiguous, block_size == 0 (backend.rs:1371-1397; CUDA
//    launchers.rs:3719-3760): query_len rows (default 1) of q, head-major
//    as the CPU backend's host FA2 path reads them (attention_provider.rs:
//    251-385), against keys 0..past_len of K/V inputs 1 and 2: causal
//    (attention_mode 0) up to key past_len + 1 - query_len + row, the last
//    `window` of those when windowed; otherwise keys within `window` of the
//    row index (all keys without a window).  One row reduces to the decode
//    form: the last `window` keys when causal, the first ones otherwise;
//  * canvas, attention_mode 1 with five inputs (backend.rs:1412-1535; CUDA
//    launchers.rs:3270-3333): query_len rows, each attending the prefix keys
//    [past_len - window, past_len) of inputs 1 and 2 and every canvas key of
//    inputs 3 and 4.  A paged prefix (block_size > 0 with a paged context) is
//    not served (-10).
void launch_attention_f32kv(State &st, const FellmOpAttrs &a, const FellmTensorRef *in, uint32_t n_in,
                            FellmTensorMut *out, bool canvas) {
    if (n_in < 3) fail(FELLM_ERR_ARITY);
    for (uint32_t i = 0; i < n_in && i < 5; ++i)
        if (in[i].dtype != FELLM_DTYPE_F32) fail(FELLM_ERR_DTYPE);
    if (out[0].dtype != FELLM_DTYPE_F32) fail(FELLM_ERR_DTYPE);
    const size_t nh = a.n_heads ? a.n_heads : 1, nkv = a.n_kv_heads ? a.n_kv_heads : 1, hd = a.head_dim;
    if (!hd) fail(FELLM_ERR_SHAPE);
    const size_t kvw = nkv * hd, past = a.past_len, window = a.attention_window;
    const size_t rows = a.query_len ? a.query_len : 1;
    const size_t qn = elems(in[0], FELLM_DTYPE_F32);
    if (qn != rows * nh * hd || elems(out[0], FELLM_DTYPE_F32) != qn) fail(FELLM_ERR_SHAPE);
    size_t b1 = 0, e1 = 0, n_prefix_rows = 0, n2 = 0;
    if (canvas) {
        FellmPagedKvSnapshot snap;
        if (a.block_size > 0 && snapshot(st, snap)) fail(FELLM_ERR_DTYPE);  // paged prefix
        if (elems(in[3], FELLM_DTYPE_F32) < rows * kvw || elems(in[4], FELLM_DTYPE_F32) < rows * kvw)
            fail(FELLM_ERR_SHAPE);
        if (past && (elems(in[1], FELLM_DTYPE_F32) < past * kvw || elems(in[2], FELLM_DTYPE_F32) < past * kvw))
            fail(FELLM_ERR_SHAPE);
        b1 = window ? (past > window ? past - window : 0) : 0;
        e1 = past;
        n_prefix_rows = past;
        n2 = rows;
    } else {
        // Keys 0..past_len; query_len rows (q and out head-major), causal
        // with the rows ending at the last key, or windowed around the row
        // index when not causal (attention_provider.rs:306-318).
        const size_t seq = past + 1;
        if (elems(in[1], FELLM_DTYPE_F32) < seq * kvw || elems(in[2], FELLM_DTYPE_F32) < seq * kvw)
            fail(FELLM_ERR_SHAPE);
        const bool causal = a.attention_mode == 0;
        if (causal && seq < rows) fail(FELLM_ERR_SHAPE);
        void *q = ensure_input(st, in[0]);
        void *k = ensure_input_prefix(st, in[1], seq * kvw * 4);
        void *v = ensure_input_prefix(st, in[2], seq * kvw * 4);
        void *o = ensure_output(st, out[0]);
        check(fellm_rocm_attention_f32kv_rows((const float *)q, (float *)o, (uint32_t)rows, (uint32_t)nh,
                                              (uint32_t)nkv, (uint32_t)hd, (const float *)k, (const float *)v,
                                              (uint32_t)seq, a.scale, causal ? 1u : 0u, (uint32_t)window,
                                              stream_ptr(st)));
        finish_outputs(st, out, 1);
        return;
    }
    void *q = ensure_input(st, in[0]);
    void *k1 = nullptr, *v1 = nullptr, *k2 = nullptr, *v2 = nullptr;
    // Only the rows read are uploaded.  The mirrors are keyed by the whole
    // K/V tensors, so each decode step uploads just the rows appended since
    // the last one, and _fellm_plugin_invalidate_f32 over the tensor (after a
    // host rewrite) reaches them.  The CUDA plugin keys a mirror per prefix
    // slice instead (launchers.rs:3719-3760), which allocates and uploads the
    // whole prefix again at every step.
    if (n_prefix_rows) {
        k1 = ensure_input_prefix(st, in[1], n_prefix_rows * kvw * 4);
        v1 = ensure_input_prefix(st, in[2], n_prefix_rows * kvw * 4);
    }
    if (n2) {
        k2 = ensure_input_prefix(st, in[3], n2 * kvw * 4);
        v2 = ensure_input_prefix(st, in[4], n2 * kvw * 4);
    }
    void *o = ensure_output(st, out[0]);
    check(fellm_rocm_attention_f32kv((const float *)q, (float *)o, (uint32_t)rows, (uint32_t)nh, (uint32_t)nkv,
                                     (uint32_t)hd, (const float *)k1, (const float *)v1, (uint32_t)b1, (uint32_t)e1,
                                     (const float *)k2, (const float *)v2, (uint32_t)n2, a.scale, stream_ptr(st)));
    finish_outputs(st, out, 1);
}

int launch_attention(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                     uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 1, 1, true, [&](State &st) {
        const FellmOpAttrs &a = *attrs;
        const bool canvas = a.attention_mode == 1 && n_in >= 5;
        if (canvas || a.block_size == 0) {
            launch_attention_f32kv(st, a, in, n_in, out, canvas);
            return;
        }
        FellmPagedKvSnapshot snap;
        if (!snapshot(st, snap)) fail(FELLM_ERR_PAGED_MISSING);
        const uint32_t dt = in[0].dtype, odt = out[0].dtype;
        const size_t nh = a.n_heads ? a.n_heads : 1, nkv = a.n_kv_heads ? a.n_kv_heads : 1, hd = a.head_dim;
        if (!hd) fail(FELLM_ERR_SHAPE);
        const size_t width = nh * hd, qn = elems(in[0], dt);
        const bool batched = snap.batch_size > 1 || qn > width;
        const size_t batch = batched ? snap.batch_size : 1;
        if (qn != batch * width || elems(out[0], odt) != qn) fail(FELLM_ERR_SHAPE);
        std::vector<uint32_t> lens(batch);
        // One decode row attends to the step block's sequence_length keys
        // when there is a step block (launchers.rs:3495-3660), which a replay
        // can advance; its key range is then sized for the whole table.
        const uint32_t *step_len = batched ? nullptr : step_u32(st, 2);
        if (batched) {
            if (!snap.row_lengths) fail(FELLM_ERR_PAGED_MISSING);
            std::memcpy(lens.data(), snap.row_lengths, batch * 4);
        } else {
            lens[0] = a.past_len + 1;
        }
        uint32_t max_seq = 1;
        for (uint32_t v : lens) max_seq = v > max_seq ? v : max_seq;
        const uint32_t causal = batched ? 1u : (a.attention_mode == 0 ? 1u : 0u);
        const uint32_t kv_dt = a.cast_to == FELLM_DTYPE_BF16 ? FELLM_DTYPE_BF16 : FELLM_DTYPE_F16;
        void *q = ensure_input(st, in[0]);
        const uint32_t *len_dev = nullptr;
        FellmRocmPagedKv kv = paged_geometry(st, snap, a.layer_ord, kv_dt, step_len ? nullptr : lens.data(), &len_dev,
                                             nullptr, nullptr, batch);
        if (step_len) {
            len_dev = step_len;
            const uint64_t cap = (uint64_t)kv.n_logical_blocks * kv.block_size;
            max_seq = cap > 0xffffffffull ? 0xffffffffu : (uint32_t)cap;
        }
        const uint64_t ws = fellm_rocm_paged_attention_workspace((uint32_t)batch, (uint32_t)nh, (uint32_t)nkv,
                                                                 (uint32_t)hd, max_seq);
        if (ws) ensure_capacity(st.attn_ws, ws);
        void *o = ensure_output(st, out[0]);
        check(fellm_rocm_paged_attention(q, dt, o, odt, (uint32_t)batch, (uint32_t)nh, (uint32_t)nkv, (uint32_t)hd,
                                         len_dev, max_seq, a.scale, causal,
                                         a.attention_window, &kv, ws ? static_cast<float *>(st.attn_ws.dev) : nullptr,
                                         ws, stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

void check_ids(const FellmTensorRef &ids_t, uint64_t vocab, std::vector<uint32_t> &ids) {
    if (ids_t.dtype != FELLM_DTYPE_U32 || !ids_t.data || ids_t.byte_len == 0 || ids_t.byte_len % 4) fail(FELLM_ERR_SHAPE);
    ids.resize(ids_t.byte_len / 4);
    std::memcpy(ids.data(), ids_t.data, ids_t.byte_len);
    for (uint32_t id : ids)
        if (id >= vocab) fail(FELLM_ERR_SHAPE);  // CPU panics on out-of-range rows; CUDA returns -2
}

// Ids of an embedding launch.  One id with a step block: the device address
// of the block's token_id (embedding_*_row, launchers.rs:1225-1260), and the
// host value is not read (an out-of-range device id gives a zero row).
// Otherwise the host ids, validated, and NULL (stage them).
const void *single_id(State &st, const FellmTensorRef &ids_t, uint64_t vocab, std::vector<uint32_t> &ids) {
    if (ids_t.dtype == FELLM_DTYPE_U32 && ids_t.byte_len == 4)
        if (const uint32_t *p = step_u32(st, 0)) {
            ids.assign(1, 0);
            return p;
        }
    check_ids(ids_t, vocab, ids);
    return nullptr;
}

const void *stage_ids(State &st, const std::vector<uint32_t> &ids) {
    std::vector<void *> staged;
    stage_small(st, {ids.data()}, {ids.size() * 4}, staged);
    return staged[0];
}

uint64_t table_row_bytes(uint32_t dt, uint64_t dim) {
    switch (dt) {
        case FELLM_DTYPE_Q4K: return dim % 256 ? 0 : dim / 256 * 144;
        case FELLM_DTYPE_Q5K: return dim % 256 ? 0 : dim / 256 * 176;
        case FELLM_DTYPE_Q6K: return dim % 256 ? 0 : dim / 256 * 210;
        case FELLM_DTYPE_Q8_0: return dim % 32 ? 0 : dim / 32 * 34;
        default: return dim * dtype_size(dt);
    }
}

// Embedding [table, ids] -> rows (backend.rs:1026-1046).
int launch_embedding(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                     uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 2, 1, false, [&](State &st) {
        const FellmTensorRef &w = in[0];
        if (w.rank < 2) fail(FELLM_ERR_SHAPE);
        const uint64_t vocab = w.dims[0], dim = w.dims[1];
        const uint64_t rb = table_row_bytes(w.dtype, dim);
        if (!rb || w.byte_len < vocab * rb || dim > 0xffffffffull) fail(FELLM_ERR_SHAPE);
        std::vector<uint32_t> ids;
        const void *idd = single_id(st, in[1], vocab, ids);
        const uint32_t odt = out[0].dtype;
        if (elems(out[0], odt) != ids.size() * dim) fail(FELLM_ERR_SHAPE);
        void *table = ensure_input(st, w);
        if (!idd) idd = stage_ids(st, ids);
        void *o = ensure_output(st, out[0]);
        check(fellm_rocm_embedding(table, w.dtype, vocab, (uint32_t)dim, (const uint32_t *)idd, (uint32_t)ids.size(), o,
                                   odt, nullptr, stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

// Custom rocm:embedding_rmsnorm [table, ids, w] -> [h, y]; attrs.eps.
int launch_embedding_rmsnorm(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                             uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 3, 2, true, [&](State &st) {
        const FellmTensorRef &w = in[0];
        if (w.rank < 2) fail(FELLM_ERR_SHAPE);
        const uint64_t vocab = w.dims[0], dim = w.dims[1];
        const uint64_t rb = table_row_bytes(w.dtype, dim);
        if (!rb || w.byte_len < vocab * rb || dim > 0xffffffffull) fail(FELLM_ERR_SHAPE);
        std::vector<uint32_t> ids;
        const void *idd = single_id(st, in[1], vocab, ids);
        if (in[2].dtype != FELLM_DTYPE_F32 || elems(in[2], FELLM_DTYPE_F32) != dim) fail(FELLM_ERR_SHAPE);
        const uint32_t odt = out[0].dtype;
        if (out[1].dtype != odt || elems(out[0], odt) != ids.size() * dim || elems(out[1], odt) != ids.size() * dim)
            fail(FELLM_ERR_SHAPE);
        void *table = ensure_input(st, w);
        if (!idd) idd = stage_ids(st, ids);
        void *nw = ensure_input(st, in[2]);
        void *h = ensure_output(st, out[0]);
        void *y = ensure_output(st, out[1]);
        check(fellm_rocm_embedding_rmsnorm(table, w.dtype, vocab, (uint32_t)dim, (const uint32_t *)idd,
                                           (uint32_t)ids.size(), (const float *)nw, attrs->eps, h, y, odt, nullptr,
                                           stream_ptr(st)));
        finish_outputs(st, out, 2);
    });
}

// Custom rocm:router_topk [logits f32 [T, E]] -> [ids u32 [T, k], weights f32 [T, k]].
int launch_router_topk(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                       uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 1, 2, true, [&](State &st) {
        const FellmOpAttrs &a = *attrs;
        if (in[0].dtype != FELLM_DTYPE_F32 || out[0].dtype != FELLM_DTYPE_U32 || out[1].dtype != FELLM_DTYPE_F32)
            fail(FELLM_ERR_DTYPE);
        const size_t n = elems(in[0], FELLM_DTYPE_F32), e = a.n_experts;
        if (!e || n % e) fail(FELLM_ERR_SHAPE);
        const size_t tokens = n / e;
        const size_t k = a.n_expert_used < e ? a.n_expert_used : e;
        if (elems(out[0], FELLM_DTYPE_U32) != tokens * k || elems(out[1], FELLM_DTYPE_F32) != tokens * k)
            fail(FELLM_ERR_SHAPE);
        void *l = ensure_input(st, in[0]);
        void *ids = ensure_output(st, out[0]);
        void *wts = ensure_output(st, out[1]);
        check(fellm_rocm_router_topk((const float *)l, (uint32_t)tokens, (uint32_t)e, a.n_expert_used,
                                     a.expert_gating_func, a.norm_topk_prob, a.routed_scaling_factor,
                                     (uint32_t *)ids, (float *)wts, stream_ptr(st)));
        finish_outputs(st, out, 2);
    });
}

uint64_t kquant_row_bytes(uint32_t dt, uint64_t cols) {
    if (cols % 256) return 0;
    switch (dt) {
        case FELLM_DTYPE_Q4K: return cols / 256 * 144;
        case FELLM_DTYPE_Q5K: return cols / 256 * 176;
        case FELLM_DTYPE_Q6K: return cols / 256 * 210;
        default: return 0;
    }
}

// GateUpSwiGlu [gate_w, up_w, x] -> out (backend.rs:944-1002; the CUDA
// plugin's launch_q4k_gate_up_swiglu, launchers.rs:1654-1744): weights
// [rows, cols] K-quant, x f32 [cols], out f32 [rows].
int launch_gate_up_swiglu(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                          uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 3, 1, false, [&](State &st) {
        const FellmTensorRef &g = in[0], &u = in[1];
        if (in[2].dtype != FELLM_DTYPE_F32 || out[0].dtype != FELLM_DTYPE_F32) fail(FELLM_ERR_DTYPE);
        if (g.rank != 2 || u.rank != 2 || g.dims[0] != u.dims[0] || g.dims[1] != u.dims[1]) fail(FELLM_ERR_SHAPE);
        const uint64_t rows = g.dims[0], cols = g.dims[1];
        const uint64_t grb = kquant_row_bytes(g.dtype, cols), urb = kquant_row_bytes(u.dtype, cols);
        if (!grb || !urb) fail(g.dtype == FELLM_DTYPE_Q4K || g.dtype == FELLM_DTYPE_Q5K || g.dtype == FELLM_DTYPE_Q6K
                                   ? FELLM_ERR_SHAPE
                                   : FELLM_ERR_DTYPE);
        if (g.byte_len < rows * grb || u.byte_len < rows * urb || rows > 0xffffffffull) fail(FELLM_ERR_SHAPE);
        if (elems(in[2], FELLM_DTYPE_F32) != cols || elems(out[0], FELLM_DTYPE_F32) != rows) fail(FELLM_ERR_SHAPE);
        void *gw = ensure_input(st, g);
        void *uw = ensure_input(st, u);
        void *x = ensure_input(st, in[2]);
        void *o = ensure_output(st, out[0]);
        check(fellm_rocm_gate_up_swiglu(gw, g.dtype, uw, u.dtype, (uint32_t)rows, (uint32_t)cols, (const float *)x,
                                        (float *)o, stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

// Cast [x] -> y of another dtype, on the device: the CPU backend's
// conversions (backend.rs:1603-1667, fellm_rocm_cast).  y stays device-valid
// like every other output (materialise it with a same-dtype Cast).
int launch_cast_convert(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                        uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 1, 1, false, [&](State &st) {
        const uint32_t sdt = in[0].dtype, ddt = out[0].dtype;
        const size_t n = elems(out[0], ddt);
        const bool quant = sdt == FELLM_DTYPE_Q4K || sdt == FELLM_DTYPE_Q5K || sdt == FELLM_DTYPE_Q6K ||
                           sdt == FELLM_DTYPE_Q8_0;
        const size_t need = quant ? table_row_bytes(sdt, n) : n * dtype_size(sdt);
        if (!need || in[0].byte_len < need) fail(FELLM_ERR_SHAPE);
        void *src = ensure_input(st, in[0]);
        void *dst = ensure_output(st, out[0]);
        check(fellm_rocm_cast(src, sdt, dst, ddt, n, stream_ptr(st)));
        finish_outputs(st, out, 1);
    });
}

// Cast [x] -> host x of the same dtype: materialise a device-valid mirror into
// host storage (launchers.rs:140-170).
int launch_materialize(const FellmOpAttrs *attrs, const FellmTensorRef *in, uint32_t n_in, FellmTensorMut *out,
                       uint32_t n_out, FellmStreamHandle) {
    return guarded(attrs, in, n_in, out, n_out, 1, 1, false, [&](State &st) {
        if (in[0].byte_len != out[0].byte_len || !out[0].data) fail(FELLM_ERR_SHAPE);
        if (in[0].dtype != out[0].dtype) fail(FELLM_ERR_DTYPE);
        void *src = ensure_input(st, in[0]);
        hip_check(hipMemcpyAsync(out[0].data, src, out[0].byte_len, hipMemcpyDeviceToHost, stream_locked(st)));
        hip_check(hipStreamSynchronize(stream_locked(st)), FELLM_ERR_ALLOC);
    });
}

const char kManifest[] =
    "{\"schema\":1,\"id\":\"fellm.rocm\",\"name\":\"FeLLM ROCm gfx950 kernels\",\"version\":\"0.1.0\","
    "\"provides\":[{\"type\":\"backend\",\"id\":\"rocm\"},{\"type\":\"kernels\",\"backend\":\"rocm\"}]}";

int register_one(FellmKernelRegistryVtable *vt, uint32_t op, std::initializer_list<uint32_t> ins, uint32_t out,
                 FellmPluginLaunchFn fn) {
    FellmPluginOpRegistration reg;
    std::memset(&reg, 0, sizeof(reg));
    reg.op_kind = op;
    reg.n_input_dtypes = (uint32_t)ins.size();
    uint32_t i = 0;
    for (uint32_t d : ins) reg.input_dtypes[i++] = d;
    reg.output_dtype = out;
    reg.launch = fn;
    return vt->register_op(vt->registry, &reg);
}

}  // namespace

extern "C" {

FellmAbiVersion _fellm_plugin_abi_version(void) { return FellmAbiVersion{0, 9, 0}; }

FellmPluginManifestJson _fellm_plugin_manifest_json(void) {
    return FellmPluginManifestJson{reinterpret_cast<const uint8_t *>(kManifest), sizeof(kManifest) - 1};
}

int _fellm_plugin_init(const FellmHostContext *ctx) {
    try {
        if (!ctx) return FELLM_ERR_ARITY;
        State &st = state();
        std::lock_guard<std::mutex> lock(st.mu);
        st.ctx = *ctx;
        st.have_ctx = true;
        return FELLM_OK;  // device work is deferred to the first launch
    } catch (...) {
        return FELLM_ERR_PANIC;
    }
}

int _fellm_plugin_register_kernels(FellmKernelRegistryVtable *vt) {
    try {
        if (!vt || !vt->register_op) return FELLM_ERR_ARITY;
        const uint32_t F32 = FELLM_DTYPE_F32, F16 = FELLM_DTYPE_F16, BF16 = FELLM_DTYPE_BF16;
        const uint32_t Q4K = FELLM_DTYPE_Q4K, Q5K = FELLM_DTYPE_Q5K, Q6K = FELLM_DTYPE_Q6K, U32 = FELLM_DTYPE_U32;
        const uint32_t Q8_0 = FELLM_DTYPE_Q8_0;
        struct R {
            uint32_t op;
            std::initializer_list<uint32_t> ins;
            uint32_t out;
            FellmPluginLaunchFn fn;
        };
        const R regs[] = {
            // Reference keys (plugins/cuda_kernels/src/lib.rs:337-720).
            {FELLM_OP_CAST, {F32}, F32, launch_materialize},
            // Same-dtype Cast = materialise a device-valid mirror into host memory.
            {FELLM_OP_CAST, {F16}, F16, launch_materialize},
            {FELLM_OP_CAST, {BF16}, BF16, launch_materialize},
            {FELLM_OP_CAST, {U32}, U32, launch_materialize},
            {FELLM_OP_CAST, {F16}, F32, launch_cast_convert},
            {FELLM_OP_CAST, {BF16}, F32, launch_cast_convert},
            {FELLM_OP_CAST, {F32}, F16, launch_cast_convert},
            {FELLM_OP_CAST, {F32}, BF16, launch_cast_convert},
            {FELLM_OP_CAST, {Q4K}, F32, launch_cast_convert},
            {FELLM_OP_CAST, {Q6K}, F32, launch_cast_convert},
            {FELLM_OP_CAST, {Q5K}, F32, launch_cast_convert},
            {FELLM_OP_CAST, {Q8_0}, F32, launch_cast_convert},
            {FELLM_OP_RMSNORM, {F32, F32}, F32, launch_rmsnorm},
            {FELLM_OP_SILU_GATE, {F32, F32}, F32, launch_silu_gate},
            {FELLM_OP_ROPE, {F32, F32}, F32, launch_rope},
            {FELLM_OP_KV_WRITE, {F32, F32}, F32, launch_kv_write},
            {FELLM_OP_ADD, {F32, F32}, F32, launch_add},
            {FELLM_OP_EMBEDDING, {F32, U32}, F32, launch_embedding},
            {FELLM_OP_EMBEDDING, {BF16, U32}, F32, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q4K, U32}, F32, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q6K, U32}, F32, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q5K, U32}, F32, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q8_0, U32}, F32, launch_embedding},
            // backend-cpu also serves F16 tables (backend.rs:453-467).
            {FELLM_OP_EMBEDDING, {F16, U32}, F32, launch_embedding},
            // 16-bit activation variants.
            {FELLM_OP_RMSNORM, {F16, F32}, F16, launch_rmsnorm},
            {FELLM_OP_RMSNORM, {BF16, F32}, BF16, launch_rmsnorm},
            {FELLM_OP_SILU_GATE, {F16, F16}, F16, launch_silu_gate},
            {FELLM_OP_SILU_GATE, {BF16, BF16}, BF16, launch_silu_gate},
            {FELLM_OP_ROPE, {F16, F32}, F16, launch_rope},
            {FELLM_OP_ROPE, {BF16, F32}, BF16, launch_rope},
            {FELLM_OP_ADD, {F16, F16}, F16, launch_add},
            {FELLM_OP_ADD, {BF16, BF16}, BF16, launch_add},
            {FELLM_OP_KV_WRITE, {F16, F32}, F32, launch_kv_write},
            {FELLM_OP_KV_WRITE, {BF16, F32}, F32, launch_kv_write},
            {FELLM_OP_EMBEDDING, {F16, U32}, F16, launch_embedding},
            {FELLM_OP_EMBEDDING, {BF16, U32}, BF16, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q4K, U32}, F16, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q6K, U32}, F16, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q5K, U32}, F16, launch_embedding},
            {FELLM_OP_EMBEDDING, {Q8_0, U32}, F16, launch_embedding},
            // GateUpSwiGlu for every K-quant gate/up pair (backend-cpu accepts any
            // supported matvec dtype pair, backend.rs:430-435; the CUDA plugin
            // registers the same-dtype pairs, lib.rs:467-496).
            {FELLM_OP_GATE_UP_SWIGLU, {Q4K, Q4K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q5K, Q5K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q6K, Q6K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q4K, Q5K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q4K, Q6K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q5K, Q4K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q5K, Q6K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q6K, Q4K, F32}, F32, launch_gate_up_swiglu},
            {FELLM_OP_GATE_UP_SWIGLU, {Q6K, Q5K, F32}, F32, launch_gate_up_swiglu},
            // Attention (launchers.rs:3243): paged decode, contiguous decode and canvas; the CUDA
            // plugin registers [F32, F32, F32] and the five-input canvas form (lib.rs:537-546, 575-582).
            {FELLM_OP_ATTENTION, {F32, F32, F32}, F32, launch_attention},
            {FELLM_OP_ATTENTION, {F32, F32, F32, F32, F32}, F32, launch_attention},
            {FELLM_OP_ATTENTION, {F16, F16, F16}, F16, launch_attention},
            {FELLM_OP_ATTENTION, {BF16, BF16, BF16}, BF16, launch_attention},
            // Fused custom ops (OpKind::custom("rocm", ...)).
            {kOpAddRmsNorm, {F32, F32, F32}, F32, launch_add_rmsnorm},
            {kOpAddRmsNorm, {F16, F16, F32}, F16, launch_add_rmsnorm},
            {kOpAddRmsNorm, {BF16, BF16, F32}, BF16, launch_add_rmsnorm},
            {kOpRopeKvWrite, {F32, F32, F32, F32}, F32, launch_rope_kv_write},
            {kOpRopeKvWrite, {F16, F16, F16, F32}, F16, launch_rope_kv_write},
            {kOpRopeKvWrite, {BF16, BF16, BF16, F32}, BF16, launch_rope_kv_write},
            {kOpRouterTopK, {F32}, U32, launch_router_topk},
            {kOpEmbeddingRmsNorm, {F32, U32, F32}, F32, launch_embedding_rmsnorm},
            {kOpEmbeddingRmsNorm, {F16, U32, F32}, F16, launch_embedding_rmsnorm},
            {kOpEmbeddingRmsNorm, {Q4K, U32, F32}, F16, launch_embedding_rmsnorm},
            {kOpEmbeddingRmsNorm, {Q6K, U32, F32}, F16, launch_embedding_rmsnorm},
            {kOpEmbeddingRmsNorm, {Q5K, U32, F32}, F16, launch_embedding_rmsnorm},
            {kOpEmbeddingRmsNorm, {Q8_0, U32, F32}, F16, launch_embedding_rmsnorm},
        };
        int idx = 0;
        for (const R &r : regs) {
            ++idx;
            if (register_one(vt, r.op, r.ins, r.out, r.fn) != 0) return -100 - idx;
        }
        return FELLM_OK;
    } catch (...) {
        return FELLM_ERR_PANIC;
    }
}

void _fellm_plugin_shutdown(void) {
    try {
        State &st = state();
        std::lock_guard<std::mutex> lock(st.mu);
        st.have_ctx = false;
        std::memset(&st.ctx, 0, sizeof(st.ctx));
    } catch (...) {
    }
}

void _fellm_plugin_invalidate_f32(const float *ptr, size_t nbytes) {
    try {
        if (!ptr || nbytes == 0) return;
        State &st = state();
        std::lock_guard<std::mutex> lock(st.mu);
        // Every activation mirror whose host range overlaps the written one
        // goes stale; a mirror that only followed the host keeps the rows
        // before the write.
        const uintptr_t lo = reinterpret_cast<uintptr_t>(ptr), hi = lo + nbytes;
        for (auto &kv : st.act) {
            const uintptr_t a = kv.first.first, b = a + kv.first.second;
            if (b <= lo || a >= hi) continue;
            Mirror &m = kv.second;
            const size_t keep = lo > a ? lo - a : 0;
            m.valid_prefix = m.device_valid ? 0 : (m.valid_prefix < keep ? m.valid_prefix : keep);
            m.device_valid = false;
        }
    } catch (...) {
    }
}

FellmStreamHandle _fellm_plugin_device_stream(void) {
    try {
        State &st = state();
        std::lock_guard<std::mutex> lock(st.mu);
        return reinterpret_cast<FellmStreamHandle>(stream_locked(st));
    } catch (...) {
        return 0;
    }
}

int _fellm_plugin_update_step_params(const FellmDeviceStepParams *params) {
    try {
        if (!params) return FELLM_ERR_ARITY;
        State &st = state();
        std::lock_guard<std::mutex> lock(st.mu);
        st.capturing = stream_capturing(st);  // updates go between replays, not into one
        ensure_capacity(st.step_params, sizeof(FellmDeviceStepParams));
        upload(st, st.step_params.dev, params, sizeof(FellmDeviceStepParams));
        hip_check(hipStreamSynchronize(stream_locked(st)));
        st.step_valid = true;
        return FELLM_OK;
    } catch (const LaunchError &e) {
        return e.code;
    } catch (...) {
        return FELLM_ERR_PANIC;
    }
}

int _fellm_plugin_register_device_tensor(const uint8_t *host_ptr, size_t nbytes, uint64_t device_ptr) {
    try {
        if (!host_ptr || nbytes == 0 || device_ptr == 0) return FELLM_ERR_ARITY;
        State &st = state();
        std::lock_guard<std::mutex> lock(st.mu);
        st.external[{reinterpret_cast<uintptr_t>(host_ptr), nbytes}] = device_ptr;
        return FELLM_OK;
    } catch (...) {
        return FELLM_ERR_PANIC;
    }
}

const char *fellm_rocm_version(void) { return "fellm-rocm 0.1.0 gfx950"; }

}  // extern "C"

// Model runtime of libmgc_hip.so: one HBM block per model, weights uploaded once, the forward
// captured into a hipGraph on first use and replayed after, a device error flag for Gather
// (zeroed at init, cleared again only after a check finds it set).
//
// Mirrors what the reference does around its generated mgc_run (allocate the arena once,
// serialize calls, map status 1 to a Gather error: src/ml_graph_compiler/codegen/
// runtime_lib.py:44-156) for a device that sits across PCIe: inputs are staged into device
// buffers inside the same allocation, so a host call is H2D copies, one graph launch, D2H copies
// and one synchronization.
#include <string.h>

#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "mgc_device.h"

namespace {

std::mutex g_err_mutex;
std::string g_last_error;

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

struct ModelState {
    hipStream_t stream = nullptr;
    unsigned char *block = nullptr;
    unsigned char *A = nullptr;
    unsigned char *W = nullptr;
    std::vector<unsigned char *> in_stage, out_stage;
    int *flag = nullptr;
    mgc_hip_exec exec{};
    // graph for the staging buffers, and one for the last set of caller device pointers
    hipGraphExec_t staged_graph = nullptr;
    hipGraphExec_t device_graph = nullptr;
    std::vector<const void *> device_key;
    std::vector<double> prof;
    std::vector<hipEvent_t> ev_b, ev_e;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    int host_flag = 0;
};

int fail(const char *where, hipError_t err) {
    mgc::set_error(where, err);
    return MGC_ERR_HIP;
}

#define MGC_CHECK(call)                                                                        \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) return fail(#call, e_);                                          \
    } while (0)

ModelState *state(mgc_hip_model *m) { return static_cast<ModelState *>(m->state); }

// Enqueue one forward pass on the model stream. The Gather error flag is not cleared here: it
// is zero from init and only a bad index sets it, so it stays zero until finish() reads it set
// and clears it (outside any captured graph). No kernel of the replayed graph spends a launch
// on it, and an error in a forward that nobody checked is reported by the next check.
int enqueue_forward(mgc_hip_model *m, ModelState *s, const void *const *in, void *const *out) {
    s->exec.launch_error = 0;
    m->forward(&s->exec, in, out, s->A, s->W);
    if (s->exec.launch_error) return fail("kernel launch", (hipError_t)s->exec.launch_error);
    return MGC_OK;
}

int capture(mgc_hip_model *m, ModelState *s, const void *const *in, void *const *out,
            hipGraphExec_t *exec) {
    hipGraph_t graph = nullptr;
    MGC_CHECK(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_forward(m, s, in, out);
    hipError_t end = hipStreamEndCapture(s->stream, &graph);
    if (rc != MGC_OK) {
        if (graph) hipGraphDestroy(graph);
        return rc;
    }
    if (end != hipSuccess) return fail("hipStreamEndCapture", end);
    hipError_t inst = hipGraphInstantiate(exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (inst != hipSuccess) return fail("hipGraphInstantiate", inst);
    return MGC_OK;
}

int finish(ModelState *s) {
    MGC_CHECK(hipMemcpyAsync(&s->host_flag, s->flag, sizeof(int), hipMemcpyDeviceToHost,
                             s->stream));
    MGC_CHECK(hipStreamSynchronize(s->stream));
    if (!s->host_flag) return MGC_OK;
    MGC_CHECK(hipMemsetAsync(s->flag, 0, sizeof(int), s->stream));
    MGC_CHECK(hipStreamSynchronize(s->stream));
    return MGC_ERR_GATHER_INDEX;
}

int ensure_staged_graph(mgc_hip_model *m, ModelState *s) {
    if (s->staged_graph) return MGC_OK;
    std::vector<const void *> in(s->in_stage.begin(), s->in_stage.end());
    std::vector<void *> out(s->out_stage.begin(), s->out_stage.end());
    in.push_back(nullptr);
    out.push_back(nullptr);
    return capture(m, s, in.data(), out.data(), &s->staged_graph);
}

}  // namespace

namespace mgc {

void set_error(const char *where, hipError_t err) {
    std::lock_guard<std::mutex> lock(g_err_mutex);
    g_last_error = std::string(where) + ": " + hipGetErrorString(err);
}

void note_launch(mgc_hip_exec *x) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        if (!x->launch_error) x->launch_error = (int)err;
        set_error("kernel launch", err);
    }
}

}  // namespace mgc

extern "C" {

const char *mgc_hip_last_error(void) {
    std::lock_guard<std::mutex> lock(g_err_mutex);
    return g_last_error.c_str();
}

const char *mgc_hip_version(void) { return "mgc_hip 0.1 gfx950"; }

int mgc_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

mgc_hip_exec *mgc_hip_exec_create(void *stream) {
    mgc_hip_exec *x = new (std::nothrow) mgc_hip_exec();
    if (!x) return nullptr;
    x->stream = static_cast<hipStream_t>(stream);
    hipError_t err = hipMalloc((void **)&x->flag, sizeof(int));
    if (err == hipSuccess) err = hipMemset(x->flag, 0, sizeof(int));
    if (err != hipSuccess) {
        mgc::set_error("mgc_hip_exec_create", err);
        if (x->flag) hipFree(x->flag);
        delete x;
        return nullptr;
    }
    return x;
}

int mgc_hip_exec_status(mgc_hip_exec *x) {
    if (!x) return MGC_ERR_ARGS;
    const int launch = x->launch_error;
    x->launch_error = 0;
    // launchers report operands outside a kernel's limits as hipErrorInvalidValue
    if (launch) return launch == (int)hipErrorInvalidValue ? MGC_ERR_ARGS : MGC_ERR_HIP;
    int host = 0;
    MGC_CHECK(hipMemcpyAsync(&host, x->flag, sizeof(int), hipMemcpyDeviceToHost, x->stream));
    MGC_CHECK(hipStreamSynchronize(x->stream));
    if (!host) return MGC_OK;
    MGC_CHECK(hipMemsetAsync(x->flag, 0, sizeof(int), x->stream));
    MGC_CHECK(hipStreamSynchronize(x->stream));
    return MGC_ERR_GATHER_INDEX;
}

void mgc_hip_exec_destroy(mgc_hip_exec *x) {
    if (!x) return;
    if (x->flag) hipFree(x->flag);
    delete x;
}

int mgc_hip_model_init(mgc_hip_model *m, const unsigned char *weights_host, unsigned char **A,
                       unsigned char **W) {
    if (!m) return MGC_ERR_ARGS;
    if (m->state) {
        ModelState *s = state(m);
        if (A) *A = s->A;
        if (W) *W = s->W;
        return MGC_OK;
    }
    if (m->weights_bytes && !weights_host) return MGC_ERR_ARGS;
    size_t off = 0;
    size_t arena_off = off;
    off += align256(m->arena_bytes ? m->arena_bytes : 1);
    size_t weights_off = off;
    off += align256(m->weights_bytes ? m->weights_bytes : 1);
    std::vector<size_t> in_off, out_off;
    for (int i = 0; i < m->n_inputs; ++i) {
        in_off.push_back(off);
        off += align256(m->input_bytes[i] ? m->input_bytes[i] : 1);
    }
    for (int j = 0; j < m->n_outputs; ++j) {
        out_off.push_back(off);
        off += align256(m->output_bytes[j] ? m->output_bytes[j] : 1);
    }
    size_t flag_off = off;
    off += 256;

    ModelState *s = new ModelState();
    hipError_t err = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (err == hipSuccess) err = hipMalloc((void **)&s->block, off);
    if (err != hipSuccess) {
        if (s->stream) hipStreamDestroy(s->stream);
        delete s;
        return fail("mgc_hip_model_init", err);
    }
    s->A = s->block + arena_off;
    s->W = s->block + weights_off;
    for (size_t o : in_off) s->in_stage.push_back(s->block + o);
    for (size_t o : out_off) s->out_stage.push_back(s->block + o);
    s->flag = reinterpret_cast<int *>(s->block + flag_off);
    err = hipMemset(s->flag, 0, sizeof(int));
    if (err != hipSuccess) {
        hipFree(s->block);
        hipStreamDestroy(s->stream);
        delete s;
        return fail("mgc_hip_model_init", err);
    }
    if (m->weights_bytes) {
        err = hipMemcpy(s->W, weights_host, m->weights_bytes, hipMemcpyHostToDevice);
        if (err != hipSuccess) {
            hipFree(s->block);
            hipStreamDestroy(s->stream);
            delete s;
            return fail("weights upload", err);
        }
    }
    s->exec.stream = s->stream;
    s->exec.flag = s->flag;
    s->exec.n_nodes = m->n_nodes;
    s->prof.assign(m->n_nodes > 0 ? m->n_nodes : 0, 0.0);
    if (m->n_nodes > 0) {
        s->ev_b.resize(m->n_nodes);
        s->ev_e.resize(m->n_nodes);
        for (int k = 0; k < m->n_nodes; ++k) {
            hipEventCreate(&s->ev_b[k]);
            hipEventCreate(&s->ev_e[k]);
        }
        s->exec.ev_begin = s->ev_b.data();
        s->exec.ev_end = s->ev_e.data();
    }
    hipEventCreate(&s->t0);
    hipEventCreate(&s->t1);
    m->state = s;
    if (A) *A = s->A;
    if (W) *W = s->W;
    return MGC_OK;
}

static int check_ptrs(mgc_hip_model *m, unsigned char *A, const unsigned char *W) {
    if (!m || !m->state) return MGC_ERR_ARGS;
    ModelState *s = state(m);
    if (A != s->A || W != s->W) {
        mgc::set_error("mgc_run: A/W are not the pointers mgc_hip_init returned",
                       hipErrorInvalidValue);
        return MGC_ERR_ARGS;
    }
    return MGC_OK;
}

int mgc_hip_model_run(mgc_hip_model *m, const void *const *inputs, void *const *outputs,
                      unsigned char *A, const unsigned char *W) {
    int rc = check_ptrs(m, A, W);
    if (rc) return rc;
    ModelState *s = state(m);
    for (int i = 0; i < m->n_inputs; ++i)
        if (m->input_bytes[i])
            MGC_CHECK(hipMemcpyAsync(s->in_stage[i], inputs[i], m->input_bytes[i],
                                     hipMemcpyHostToDevice, s->stream));
    rc = ensure_staged_graph(m, s);
    if (rc) return rc;
    MGC_CHECK(hipGraphLaunch(s->staged_graph, s->stream));
    for (int j = 0; j < m->n_outputs; ++j)
        if (m->output_bytes[j])
            MGC_CHECK(hipMemcpyAsync(outputs[j], s->out_stage[j], m->output_bytes[j],
                                     hipMemcpyDeviceToHost, s->stream));
    return finish(s);
}

int mgc_hip_model_run_device(mgc_hip_model *m, const void *const *inputs, void *const *outputs,
                             unsigned char *A, const unsigned char *W) {
    int rc = check_ptrs(m, A, W);
    if (rc) return rc;
    ModelState *s = state(m);
    std::vector<const void *> key;
    for (int i = 0; i < m->n_inputs; ++i) key.push_back(inputs[i]);
    for (int j = 0; j < m->n_outputs; ++j) key.push_back(outputs[j]);
    if (!s->device_graph || key != s->device_key) {
        if (s->device_graph) {
            hipGraphExecDestroy(s->device_graph);
            s->device_graph = nullptr;
        }
        rc = capture(m, s, inputs, outputs, &s->device_graph);
        if (rc) return rc;
        s->device_key = key;
    }
    MGC_CHECK(hipGraphLaunch(s->device_graph, s->stream));
    return finish(s);
}

int mgc_hip_model_upload(mgc_hip_model *m, const void *const *inputs) {
    if (!m || !m->state) return MGC_ERR_ARGS;
    ModelState *s = state(m);
    for (int i = 0; i < m->n_inputs; ++i)
        if (m->input_bytes[i])
            MGC_CHECK(hipMemcpyAsync(s->in_stage[i], inputs[i], m->input_bytes[i],
                                     hipMemcpyHostToDevice, s->stream));
    MGC_CHECK(hipStreamSynchronize(s->stream));
    return MGC_OK;
}

int mgc_hip_model_launch(mgc_hip_model *m, int replays) {
    if (!m || !m->state) return MGC_ERR_ARGS;
    ModelState *s = state(m);
    int rc = ensure_staged_graph(m, s);
    if (rc) return rc;
    for (int r = 0; r < replays; ++r) MGC_CHECK(hipGraphLaunch(s->staged_graph, s->stream));
    return MGC_OK;
}

int mgc_hip_model_sync(mgc_hip_model *m) {
    if (!m || !m->state) return MGC_ERR_ARGS;
    return finish(state(m));
}

int mgc_hip_model_download(mgc_hip_model *m, void *const *outputs) {
    if (!m || !m->state) return MGC_ERR_ARGS;
    ModelState *s = state(m);
    for (int j = 0; j < m->n_outputs; ++j)
        if (m->output_bytes[j])
            MGC_CHECK(hipMemcpyAsync(outputs[j], s->out_stage[j], m->output_bytes[j],
                                     hipMemcpyDeviceToHost, s->stream));
    return finish(s);
}

double mgc_hip_model_time_graph(mgc_hip_model *m, int replays) {
    if (!m || !m->state) return -1.0;
    ModelState *s = state(m);
    if (ensure_staged_graph(m, s)) return -1.0;
    if (hipEventRecord(s->t0, s->stream) != hipSuccess) return -1.0;
    for (int r = 0; r < replays; ++r)
        if (hipGraphLaunch(s->staged_graph, s->stream) != hipSuccess) return -1.0;
    if (hipEventRecord(s->t1, s->stream) != hipSuccess) return -1.0;
    if (hipEventSynchronize(s->t1) != hipSuccess) return -1.0;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, s->t0, s->t1) != hipSuccess) return -1.0;
    return (double)ms;
}

int mgc_hip_model_profile_run(mgc_hip_model *m, int replays) {
    if (!m || !m->state) return MGC_ERR_ARGS;
    ModelState *s = state(m);
    if (m->n_nodes <= 0) return MGC_ERR_ARGS;
    std::vector<const void *> in(s->in_stage.begin(), s->in_stage.end());
    std::vector<void *> out(s->out_stage.begin(), s->out_stage.end());
    in.push_back(nullptr);
    out.push_back(nullptr);
    for (int r = 0; r < replays; ++r) {
        s->exec.profiling = 1;
        int rc = enqueue_forward(m, s, in.data(), out.data());
        s->exec.profiling = 0;
        if (rc) return rc;
        rc = finish(s);
        if (rc) return rc;
        for (int k = 0; k < m->n_nodes; ++k) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, s->ev_b[k], s->ev_e[k]) == hipSuccess)
                s->prof[k] += 1e-3 * ms;
        }
    }
    return MGC_OK;
}

const double *mgc_hip_model_profile_data(mgc_hip_model *m) {
    if (!m || !m->state) return nullptr;
    return state(m)->prof.data();
}

void mgc_hip_model_profile_reset(mgc_hip_model *m) {
    if (!m || !m->state) return;
    ModelState *s = state(m);
    for (double &v : s->prof) v = 0.0;
}

void mgc_hip_model_release(mgc_hip_model *m) {
    if (!m || !m->state) return;
    ModelState *s = state(m);
    hipStreamSynchronize(s->stream);
    if (s->staged_graph) hipGraphExecDestroy(s->staged_graph);
    if (s->device_graph) hipGraphExecDestroy(s->device_graph);
    for (hipEvent_t e : s->ev_b) hipEventDestroy(e);
    for (hipEvent_t e : s->ev_e) hipEventDestroy(e);
    if (s->t0) hipEventDestroy(s->t0);
    if (s->t1) hipEventDestroy(s->t1);
    hipFree(s->block);
    hipStreamDestroy(s->stream);
    delete s;
    m->state = nullptr;
}

void mgc_hip_node_begin(mgc_hip_exec *x, int node) {
    if (x->profiling && node >= 0 && node < x->n_nodes)
        (void)hipEventRecord(x->ev_begin[node], x->stream);
}

void mgc_hip_node_end(mgc_hip_exec *x, int node) {
    if (x->profiling && node >= 0 && node < x->n_nodes)
        (void)hipEventRecord(x->ev_end[node], x->stream);
}

}  // extern "C"

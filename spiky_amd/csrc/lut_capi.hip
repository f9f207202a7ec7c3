// lut_capi.hip -- the C ABI of include/spiky_lut.h: one manager object per
// LUT layer (the reference's LUTDataManagerF/I, spiky_cuda/lut/lut.cu), host
// validation with the reference's error texts, and dispatch to the kernels on
// the caller's HIP stream.  Nothing here synchronises the device.
#include "../../include/spiky_lut.h"
#include "lut_kernels.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_last_error;

struct ValueError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
    }
}

// A launch's status; a refused scratch layout names the launcher and the
// bytes it needed.
void check_launch(hipError_t e, const char *what) {
    std::string &why = spiky::scratch_refusal();
    if (e != hipSuccess && !why.empty()) {
        const std::string msg = std::string(what) + ": " + why;
        why.clear();
        throw std::runtime_error(msg);
    }
    check_hip(e, what);
}

// The bytes a launcher's scratch layout needs: the launcher run as a plan,
// which launches nothing.
template <typename F>
size_t planned_bytes(F &&launch, const char *what) {
    spiky::Scratch p = spiky::scratch_plan();
    check_launch(launch(p), what);
    return p.needed;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

template <typename F>
int guarded(F &&f) {
    try {
        f();
        g_last_error.clear();
        return SPIKY_OK;
    } catch (const ValueError &e) {
        g_last_error = e.what();
        return SPIKY_VALUE_ERROR;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return SPIKY_RUNTIME_ERROR;
    }
}

struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    int device = -1;
    void release() {
        if (ptr) {
            int cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(device);
            (void)hipFree(ptr);
            (void)hipSetDevice(cur);
        }
        ptr = nullptr;
        bytes = 0;
        device = -1;
    }
    // Make sure at least `need` bytes exist on the current device.
    void *ensure(size_t need) {
        int cur = 0;
        check_hip(hipGetDevice(&cur), "hipGetDevice");
        if (ptr && device == cur && bytes >= need) return ptr;
        release();
        if (need == 0) return nullptr;
        check_hip(hipMalloc(&ptr, need), "hipMalloc(scratch)");
        bytes = need;
        device = cur;
        return ptr;
    }
    // This buffer, grown to the bytes `launch` lays out, as its scratch.
    template <typename F>
    spiky::Scratch scratch_for(F &&launch, const char *what) {
        void *p = ensure(planned_bytes(launch, what));
        return spiky::scratch_run(p, p ? bytes : 0);
    }
    // Upload host data (re-uploads when the current device changed).
    void *upload(const void *host, size_t n, bool force) {
        int cur = 0;
        check_hip(hipGetDevice(&cur), "hipGetDevice");
        if (!force && ptr && device == cur && bytes == n) return ptr;
        release();
        if (n == 0) return nullptr;
        check_hip(hipMalloc(&ptr, n), "hipMalloc(connectivity)");
        bytes = n;
        device = cur;
        check_hip(hipMemcpy(ptr, host, n, hipMemcpyHostToDevice), "hipMemcpy(connectivity)");
        return ptr;
    }
};

struct OpStat {
    uint64_t count = 0;
    double total_ms = 0.0;
};

class ScopedTimer {
  public:
    ScopedTimer(std::map<std::string, OpStat> &stats, const char *name)
        : stats_(stats), name_(name), t0_(std::chrono::steady_clock::now()) {}
    ~ScopedTimer() {
        const double ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0_).count();
        OpStat &s = stats_[name_];
        s.count++;
        s.total_ms += ms;
    }

  private:
    std::map<std::string, OpStat> &stats_;
    const char *name_;
    std::chrono::steady_clock::time_point t0_;
};

}  // namespace

struct spiky_lut_manager {
    uint32_t n_inputs, n_outputs, n_detectors, n_anchors, sequence_length, positional_dim;
    uint64_t initial_synapse_capacity;
    uint32_t forward_group_size, backward_group_size;
    bool int_mode;
    double int_rescaler;
    bool ordered_sums = false;  // spiky_lut_set_ordered_sums
    uint64_t n_lookup;
    std::vector<std::vector<float>> metas;  // lr, min, max, noise, init
    int fully_connected = -1;               // -1: neurons not initialised
    bool context_active = false;            // set by the first forward (lut.cu:664-694)

    // sparse connectivity (host master copy + device copies)
    bool has_connectivity = false;
    std::vector<int64_t> syn_offsets;
    std::vector<int32_t> syn_targets;
    std::vector<int32_t> syn_neuron;  // lookup neuron of each synapse
    std::vector<int64_t> in_offsets;
    std::vector<int32_t> in_pairs;
    std::vector<uint32_t> in_order;  // outputs by descending list length, ties in output order
    std::vector<int32_t> row_pairs;  // (t, k) for synapse k of detector t's rows (uniform topology)
    uint32_t n_in_nonempty = 0;      // outputs with a non-empty list (the head of in_order)
    bool uniform = false;
    uint32_t max_groups = 0;
    uint32_t max_row = 0;  // most synapses of one lookup neuron
    uint32_t typ_row = 0;  // the median synapse count of the lookup neurons that have any
    DeviceBuffer d_syn_offsets, d_syn_targets, d_syn_neuron, d_in_offsets, d_in_pairs, d_in_order,
        d_row_pairs;
    bool dirty = true;

    // forward and backward keep separate scratch so that calls issued on
    // different streams never share a buffer
    DeviceBuffer scratch_fwd, scratch;
    std::map<std::string, OpStat> stats;

    // optional per-launch GPU timing with HIP events on the launch stream
    bool timing = false;
    struct Pending {
        const char *name;
        hipEvent_t start, stop;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> event_pool;
    std::map<std::string, OpStat> kernel_stats;

    hipEvent_t take_event() {
        if (!event_pool.empty()) {
            hipEvent_t e = event_pool.back();
            event_pool.pop_back();
            return e;
        }
        hipEvent_t e;
        check_hip(hipEventCreate(&e), "hipEventCreate");
        return e;
    }

    template <typename F>
    void timed(const char *name, hipStream_t st, F &&launch) {
        if (!timing) {
            launch();
            return;
        }
        Pending p{name, take_event(), take_event()};
        check_hip(hipEventRecord(p.start, st), "hipEventRecord");
        launch();
        check_hip(hipEventRecord(p.stop, st), "hipEventRecord");
        pending.push_back(p);
    }

    void collect() {
        for (auto &p : pending) {
            check_hip(hipEventSynchronize(p.stop), "hipEventSynchronize");
            float ms = 0.f;
            check_hip(hipEventElapsedTime(&ms, p.start, p.stop), "hipEventElapsedTime");
            OpStat &k = kernel_stats[p.name];
            k.count++;
            k.total_ms += ms;
            event_pool.push_back(p.start);
            event_pool.push_back(p.stop);
        }
        pending.clear();
    }

    void release_events() {
        for (auto &p : pending) {
            (void)hipEventDestroy(p.start);
            (void)hipEventDestroy(p.stop);
        }
        pending.clear();
        for (auto e : event_pool) (void)hipEventDestroy(e);
        event_pool.clear();
    }

    uint32_t n_entries() const { return 1u << n_anchors; }

    spiky::FcShape shape(uint32_t batch) const {
        spiky::FcShape s;
        s.batch = batch;
        s.n_inputs = n_inputs;
        s.n_outputs = n_outputs;
        s.n_detectors = n_detectors;
        s.n_anchors = n_anchors;
        s.n_entries = n_entries();
        s.dgs = backward_group_size;
        s.ogs = forward_group_size;
        s.ordered_sums = ordered_sums;
        return s;
    }

    void sync_connectivity() {
        d_syn_offsets.upload(syn_offsets.data(), syn_offsets.size() * sizeof(int64_t), dirty);
        d_syn_targets.upload(syn_targets.data(), syn_targets.size() * sizeof(int32_t), dirty);
        d_syn_neuron.upload(syn_neuron.data(), syn_neuron.size() * sizeof(int32_t), dirty);
        if (uniform) {
            d_in_offsets.upload(in_offsets.data(), in_offsets.size() * sizeof(int64_t), dirty);
            d_in_pairs.upload(in_pairs.data(), in_pairs.size() * sizeof(int32_t), dirty);
            d_in_order.upload(in_order.data(), in_order.size() * sizeof(uint32_t), dirty);
            d_row_pairs.upload(row_pairs.data(), row_pairs.size() * sizeof(int32_t), dirty);
        }
        dirty = false;
    }
};

namespace {

// Scratch of the allocation-free forward: one copy of this array per device,
// allocated with the code object and held until the process ends.  Host code
// never uses the array's name as a device address: noalloc_scratch() resolves
// each device's own copy once, with that device current, and kernels receive
// that pointer.
static __device__ __align__(256) uint8_t scratch[SPIKY_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mutex;
// Per device: the address of its copy of `scratch`, and an event recorded
// after the last eager call's final kernel, so that the next call (on any
// stream) starts only once that call has finished with the array.
struct NoallocDevice {
    void *ptr = nullptr;
    hipEvent_t done = nullptr;
    bool recorded = false;
};
NoallocDevice g_noalloc[kMaxDevices];

// Resolves the current device's array and event once (with that device
// current); the caller holds g_noalloc_mutex.
NoallocDevice &noalloc_device() {
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("device id out of range");
    NoallocDevice &d = g_noalloc[dev];
    if (!d.ptr) {
        void *p = nullptr;
        check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        check_hip(hipEventCreateWithFlags(&d.done, hipEventDisableTiming), "hipEventCreate(noalloc)");
        d.ptr = p;
    }
    return d;
}

void require_manager(const spiky_lut_manager *m) {
    if (!m) throw ValueError("null manager");
}

void require_initialized(const spiky_lut_manager *m) {
    if (m->fully_connected < 0) throw ValueError("neurons are not initialized (call initialize_neurons first)");
    if (m->fully_connected == 0 && !m->has_connectivity)
        throw ValueError("sparse connectivity is not compiled (call compile first)");
}

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ---- scratch layouts --------------------------------------------------------
// Each entry point's scratch launchers called with null pointers.  Run as a
// Plan or a Check a launcher reads no pointer and launches nothing, so these
// give exactly the layouts the entry points lay out: the entry points size
// their buffers with them, and spiky_lut_scratch_plan reports them.
hipError_t layout_fill_tm(const spiky_lut_manager *m, const spiky::FcShape &s, spiky::Scratch &x) {
    return spiky::launch_fill_tm(s, nullptr, nullptr, nullptr, m->int_mode, m->int_rescaler, x, nullptr);
}

hipError_t layout_fill_tm_i8(const spiky_lut_manager *m, const spiky::FcShape &s, spiky::Scratch &x) {
    return spiky::launch_fill_tm_i8(s, nullptr, nullptr, nullptr, nullptr, m->int_mode, m->int_rescaler, x,
                                    nullptr);
}

hipError_t layout_propagate_tm(const spiky::FcShape &s, spiky::Scratch &x) {
    return spiky::launch_propagate_tm(s, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, x,
                                      nullptr);
}

hipError_t layout_wgrad_fc(const spiky_lut_manager *m, const spiky::FcShape &s, spiky::Scratch &x) {
    return spiky::launch_wgrad_fc(s, nullptr, nullptr, nullptr, 1.0, m->int_mode, m->int_rescaler, true, x,
                                  nullptr);
}

// fp32 sums leave the outputs with empty lists as they are; int32 sums convert every output
uint32_t fill_sparse_order_len(const spiky_lut_manager *m) {
    return m->int_mode ? m->n_outputs : m->n_in_nonempty;
}

hipError_t layout_fill_sparse(const spiky_lut_manager *m, const spiky::SparseShape &s, spiky::Scratch &x) {
    return spiky::launch_fill_sparse_uniform(s, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                             fill_sparse_order_len(m), nullptr, m->int_mode, m->int_rescaler, x,
                                             nullptr);
}

hipError_t layout_wgrad_sparse(const spiky_lut_manager *m, const spiky::SparseShape &s, spiky::Scratch &x) {
    return spiky::launch_wgrad_sparse(s, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 1.0,
                                      true, m->int_mode, m->int_rescaler, x, m->syn_targets.size(), nullptr);
}

hipError_t layout_forward_seq(const spiky_lut_manager *m, const spiky::SeqShape &s, spiky::Scratch &x) {
    return spiky::launch_forward_seq(s, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, nullptr, 0.0f, m->int_mode, m->int_rescaler, x, nullptr);
}

hipError_t layout_backward_seq(const spiky_lut_manager *m, const spiky::SeqShape &s, spiky::Scratch &x) {
    return spiky::launch_backward_seq(s, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                      nullptr, nullptr, nullptr, nullptr, nullptr, 1.0, true, m->int_mode,
                                      m->int_rescaler, x, nullptr);
}

hipError_t layout_forward_product(const spiky_lut_manager *m, const spiky::ProductShape &s, spiky::Scratch &x) {
    return spiky::launch_forward_product(s, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, m->int_mode,
                                         m->int_rescaler, x, nullptr);
}

hipError_t layout_backward_product(const spiky_lut_manager *m, const spiky::ProductShape &s, spiky::Scratch &x) {
    return spiky::launch_backward_product(s, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                          nullptr, nullptr, nullptr, 1.0, m->int_mode,
                                          m->int_rescaler, x, nullptr);
}

// The fully connected backward's one scratch buffer, used in stream order:
// the table-major propagate's layout first, then the weight gradient's (whose
// bucket sort reads the transposed keys the propagate leaves at the start of
// its region).
struct FcBackwardRegions {
    bool tm = false;        // the table-major propagate runs
    size_t prop_bytes = 0;  // its region, a 256-byte multiple
    size_t wg_bytes = 0;    // the weight gradient's region after it
};

FcBackwardRegions fc_backward_regions(const spiky_lut_manager *m, const spiky::FcShape &s, bool with_wgrad) {
    FcBackwardRegions r;
    r.tm = !m->int_mode && spiky::tm_propagate_applies(s);
    if (r.tm)
        r.prop_bytes = align256(planned_bytes([&](spiky::Scratch &x) { return layout_propagate_tm(s, x); },
                                              "propagate_through_detectors_fc"));
    if (with_wgrad)
        r.wg_bytes = planned_bytes([&](spiky::Scratch &x) { return layout_wgrad_fc(m, s, x); },
                                   "gather_w_gradients_fc");
    return r;
}

}  // namespace

extern "C" {

const char *spiky_lut_last_error(void) { return g_last_error.c_str(); }

const char *spiky_lut_version(void) { return "spiky_amd-lut 0.1 (gfx950)"; }

int spiky_lut_create(uint32_t n_inputs, uint32_t n_outputs, uint32_t n_detectors,
                     uint32_t n_anchors_per_detector, uint32_t sequence_length,
                     uint32_t positional_dim, uint64_t initial_synapse_capacity,
                     uint32_t forward_group_size, uint32_t backward_group_size,
                     int summation_int32, double int_rescaler, spiky_lut_manager **out) {
    return guarded([&] {
        if (!out) throw ValueError("null output handle");
        *out = nullptr;
        // lut.cu:47-76
        if (n_inputs == 0) throw ValueError("n_inputs == 0");
        if (n_outputs == 0) throw ValueError("n_outputs == 0");
        if (n_detectors == 0) throw ValueError("n_detectors == 0");
        if (n_anchors_per_detector == 0) throw ValueError("n_anchors_per_detector == 0");
        if (sequence_length == 0) throw ValueError("sequence_length == 0");
        if (forward_group_size == 0) throw ValueError("forward_group_size == 0");
        if (forward_group_size > 2047) throw ValueError("forward_group_size > MAX_SYNAPSE_GROUP_SIZE");
        if (forward_group_size > 1024) throw ValueError("forward_group_size > LUT_RUNTIME_KERNELS_TPB");
        if (backward_group_size == 0) throw ValueError("backward_group_size == 0");
        if (backward_group_size > 2047) throw ValueError("backward_group_size > MAX_SYNAPSE_GROUP_SIZE");
        const uint32_t bits = n_anchors_per_detector +
                              (sequence_length > 1 ? n_anchors_per_detector + positional_dim : 0);
        if (bits > 30) throw ValueError("lookup index does not fit: too many anchors per detector");
        if (summation_int32 && !(int_rescaler > 0.0)) throw ValueError("int_rescaler must be > 0");
        auto *m = new spiky_lut_manager();
        m->n_inputs = n_inputs;
        m->n_outputs = n_outputs;
        m->n_detectors = n_detectors;
        m->n_anchors = n_anchors_per_detector;
        m->sequence_length = sequence_length;
        m->positional_dim = positional_dim;
        m->initial_synapse_capacity = initial_synapse_capacity;
        m->forward_group_size = forward_group_size;
        m->backward_group_size = backward_group_size;
        m->int_mode = summation_int32 != 0;
        m->int_rescaler = summation_int32 ? int_rescaler : 0.0;
        m->n_lookup = (uint64_t)n_detectors << bits;  // lut.cu:42
        *out = m;
    });
}

int spiky_lut_set_ordered_sums(spiky_lut_manager *m, int ordered) {
    return guarded([&] {
        require_manager(m);
        m->ordered_sums = ordered != 0;
    });
}

void spiky_lut_destroy(spiky_lut_manager *m) {
    if (!m) return;
    m->release_events();
    m->scratch.release();
    m->scratch_fwd.release();
    m->d_syn_offsets.release();
    m->d_syn_targets.release();
    m->d_syn_neuron.release();
    m->d_in_offsets.release();
    m->d_in_pairs.release();
    m->d_in_order.release();
    m->d_row_pairs.release();
    delete m;
}

int spiky_lut_register_synapse_meta(spiky_lut_manager *m, float learning_rate,
                                    float min_synaptic_weight, float max_synaptic_weight,
                                    float initial_noise_level, float initial_weight,
                                    uint32_t *out_meta_index) {
    return guarded([&] {
        require_manager(m);
        // lut.cu:148-206
        if (m->fully_connected >= 0)
            throw ValueError("can't register new synapse metas after neurons were initialized");
        if (learning_rate < 0.0f) throw ValueError("learning_rate < 0");
        if (learning_rate > 1.0f) throw ValueError("learning_rate > 1");
        if (m->int_mode) {
            const float recip = (float)(1.0 / 1048575.0);
            if (learning_rate > 0.0f && (learning_rate * m->int_rescaler) < recip)
                throw ValueError("too small value for 'learning_rate' (less than smallest distinguishable fraction)");
        }
        if (min_synaptic_weight > max_synaptic_weight) throw ValueError("min_synaptic_weight > max_synaptic_weight");
        if (initial_weight < min_synaptic_weight) throw ValueError("initial_weight < min_synaptic_weight");
        if (initial_weight > max_synaptic_weight) throw ValueError("initial_weight > max_synaptic_weight");
        std::vector<float> meta = {learning_rate, min_synaptic_weight, max_synaptic_weight,
                                   initial_noise_level, initial_weight};
        for (size_t i = 0; i < m->metas.size(); i++) {
            if (m->metas[i] == meta) {
                if (out_meta_index) *out_meta_index = (uint32_t)i;
                return;
            }
        }
        if (m->metas.size() >= 256) throw ValueError("too many different synapse metas");
        m->metas.push_back(meta);
        if (out_meta_index) *out_meta_index = (uint32_t)(m->metas.size() - 1);
    });
}

int spiky_lut_initialize_neurons(spiky_lut_manager *m, int is_fully_connected) {
    return guarded([&] {
        require_manager(m);
        if (m->metas.empty()) throw ValueError("no synapse metas were registered");
        if (is_fully_connected && m->metas.size() > 1)
            throw ValueError("fully connected mode is not compatible with multiple synapse metas");
        m->fully_connected = is_fully_connected ? 1 : 0;
    });
}

uint64_t spiky_lut_n_lookup_neurons(const spiky_lut_manager *m) { return m ? m->n_lookup : 0; }

uint64_t spiky_lut_weights_dimension(const spiky_lut_manager *m) {
    if (!m) return 0;
    if (m->fully_connected == 1) return m->n_lookup * m->n_outputs;
    return m->has_connectivity ? (uint64_t)m->syn_targets.size() : 0;
}

uint32_t spiky_lut_max_forward_groups_per_neuron(const spiky_lut_manager *m) {
    if (!m) return 0;
    if (m->fully_connected == 1)
        return (m->n_outputs + m->forward_group_size - 1) / m->forward_group_size;  // lut.cu:225
    return m->max_groups;
}

uint64_t spiky_lut_n_synapses(const spiky_lut_manager *m) {
    if (!m) return 0;
    if (m->fully_connected == 1) return 0;  // lut.cu n_synapses stays 0 in FC mode
    return (uint64_t)m->syn_targets.size();
}

int spiky_lut_set_sparse_connectivity(spiky_lut_manager *m, const int64_t *syn_offsets,
                                      const int32_t *syn_targets, uint64_t n_synapses) {
    return guarded([&] {
        require_manager(m);
        if (m->fully_connected != 0) throw ValueError("can't add lookup connections in fully connected mode");
        if (!syn_offsets || (n_synapses && !syn_targets)) throw ValueError("null connectivity arrays");
        const uint64_t nl = m->n_lookup;
        if (syn_offsets[0] != 0 || (uint64_t)syn_offsets[nl] != n_synapses)
            throw ValueError("syn_offsets must start at 0 and end at n_synapses");
        uint32_t max_groups = 0;
        int64_t max_row = 0;
        for (uint64_t n = 0; n < nl; n++) {
            const int64_t len = syn_offsets[n + 1] - syn_offsets[n];
            if (len < 0) throw ValueError("syn_offsets must be non-decreasing");
            max_groups = std::max<uint32_t>(
                max_groups, (uint32_t)((len + m->forward_group_size - 1) / m->forward_group_size));
            max_row = std::max(max_row, len);
        }
        for (uint64_t s = 0; s < n_synapses; s++)
            if (syn_targets[s] < 0 || (uint32_t)syn_targets[s] >= m->n_outputs)
                throw ValueError("synapse target out of range");
        m->syn_offsets.assign(syn_offsets, syn_offsets + nl + 1);
        m->syn_targets.assign(syn_targets, syn_targets + n_synapses);
        m->syn_neuron.assign(n_synapses, 0);
        for (uint64_t n = 0; n < nl; n++)
            for (int64_t s = syn_offsets[n]; s < syn_offsets[n + 1]; s++) m->syn_neuron[s] = (int32_t)n;
        m->max_groups = max_groups;
        m->max_row = (uint32_t)std::min<int64_t>(max_row, UINT32_MAX);
        {
            std::vector<int64_t> lens;
            lens.reserve(nl);
            for (uint64_t n = 0; n < nl; n++)
                if (syn_offsets[n + 1] > syn_offsets[n]) lens.push_back(syn_offsets[n + 1] - syn_offsets[n]);
            int64_t typ = 0;
            if (!lens.empty()) {
                std::nth_element(lens.begin(), lens.begin() + lens.size() / 2, lens.end());
                typ = lens[lens.size() / 2];
            }
            m->typ_row = (uint32_t)std::min<int64_t>(typ, UINT32_MAX);
        }
        // uniform topology: all lookup neurons of a detector share one ordered target list
        const uint32_t E = (uint32_t)(m->n_lookup / m->n_detectors);  // rows of a table
        bool uniform = true;
        for (uint32_t t = 0; t < m->n_detectors && uniform; t++) {
            const uint64_t n0 = (uint64_t)t * E;
            const int64_t len0 = syn_offsets[n0 + 1] - syn_offsets[n0];
            for (uint32_t e = 1; e < E && uniform; e++) {
                const uint64_t n = n0 + e;
                if (syn_offsets[n + 1] - syn_offsets[n] != len0) { uniform = false; break; }
                if (std::memcmp(syn_targets + syn_offsets[n], syn_targets + syn_offsets[n0],
                                (size_t)len0 * sizeof(int32_t)) != 0)
                    uniform = false;
            }
        }
        // the output-major index addresses synapses with 32-bit offsets
        if (n_synapses >= (1ull << 31)) uniform = false;
        m->uniform = uniform;
        m->in_offsets.clear();
        m->in_pairs.clear();
        m->in_order.clear();
        m->row_pairs.clear();
        m->n_in_nonempty = 0;
        if (uniform) {
            std::vector<int64_t> cnt(m->n_outputs + 1, 0);
            for (uint32_t t = 0; t < m->n_detectors; t++) {
                const uint64_t n0 = (uint64_t)t * E;
                for (int64_t s = syn_offsets[n0]; s < syn_offsets[n0 + 1]; s++) cnt[syn_targets[s] + 1]++;
            }
            for (uint32_t j = 0; j < m->n_outputs; j++) cnt[j + 1] += cnt[j];
            m->in_offsets = cnt;
            // entry p: {t, offset of synapse k of the detector's row 0, synapses a row, 0}; the
            // neurons of a detector have equal lengths, so row e's synapse k is at
            // offset + e * length
            m->in_pairs.assign((size_t)cnt[m->n_outputs] * 4, 0);
            std::vector<int64_t> pos(cnt.begin(), cnt.end() - 1);
            for (uint32_t t = 0; t < m->n_detectors; t++) {
                const uint64_t n0 = (uint64_t)t * E;
                const int64_t len0 = syn_offsets[n0 + 1] - syn_offsets[n0];
                for (int64_t s = syn_offsets[n0]; s < syn_offsets[n0 + 1]; s++) {
                    const int64_t p = pos[syn_targets[s]]++;
                    m->in_pairs[4 * p] = (int32_t)t;
                    m->in_pairs[4 * p + 1] = (int32_t)s;
                    m->in_pairs[4 * p + 2] = (int32_t)len0;
                }
            }
            // the sample-lane forward's order: longest lists first
            m->in_order.resize(m->n_outputs);
            for (uint32_t j = 0; j < m->n_outputs; j++) m->in_order[j] = j;
            std::stable_sort(m->in_order.begin(), m->in_order.end(), [&](uint32_t a, uint32_t b) {
                return cnt[a + 1] - cnt[a] > cnt[b + 1] - cnt[b];
            });
            for (uint32_t j = 0; j < m->n_outputs; j++) m->n_in_nonempty += cnt[j + 1] > cnt[j] ? 1u : 0u;
            // the weight gradient's threads: synapse k of each detector's rows
            for (uint32_t t = 0; t < m->n_detectors; t++) {
                const uint64_t n0 = (uint64_t)t * E;
                for (int64_t k = 0; k < syn_offsets[n0 + 1] - syn_offsets[n0]; k++) {
                    m->row_pairs.push_back((int32_t)t);
                    m->row_pairs.push_back((int32_t)k);
                }
            }
        }
        m->has_connectivity = true;
        m->dirty = true;
    });
}

int spiky_lut_forward_step(spiky_lut_manager *m, const float *weights, uint32_t batch_size,
                           const float *input, const int32_t *anchors, float *output,
                           int32_t *lookup_indices, float cmp_eps, float *min_deltas,
                           int32_t *min_delta_indices, void *stream) {
    return guarded([&] {
        require_manager(m);
        if (batch_size == 0) throw ValueError("batch_size == 0");
        if (m->sequence_length != 1)
            throw ValueError("forward_step should only be called when sequence_length == 1");
        require_initialized(m);
        if (!weights || !input || !anchors || !output || !lookup_indices)
            throw ValueError("null tensor pointer");
        if ((min_deltas == nullptr) != (min_delta_indices == nullptr))
            throw ValueError("w_min_anchor_deltas and w_min_anchor_delta_indices must be given together");
        ScopedTimer timer(m->stats, min_deltas ? "lut::runtime::forward_non_seq"
                                               : "lut::runtime::forward_non_seq_eval");
        m->context_active = true;
        const hipStream_t st = as_stream(stream);
        const spiky::FcShape s = m->shape(batch_size);
        m->timed("check_detectors", st, [&] {
            check_hip(spiky::launch_check_detectors(s, input, anchors, cmp_eps, lookup_indices,
                                                    min_deltas, min_delta_indices, st),
                      "check_detectors");
        });
        if (m->fully_connected == 1) {
            if (spiky::tm_fill_applies(s, m->int_mode)) {
                spiky::Scratch scr = m->scratch_fwd.scratch_for(
                    [&](spiky::Scratch &x) { return layout_fill_tm(m, s, x); }, "fill_outputs_fc");
                m->timed("fill_outputs_fc", st, [&] {
                    check_launch(spiky::launch_fill_tm(s, weights, lookup_indices, output, m->int_mode,
                                                       m->int_rescaler, scr, st),
                                 "fill_outputs_fc");
                });
            } else {
                m->timed("fill_outputs_fc", st, [&] {
                    check_hip(spiky::launch_fill_fc_f32(s, weights, lookup_indices, output,
                                                        m->int_mode, m->int_rescaler, st),
                              "fill_outputs_fc");
                });
            }
        } else {
            m->sync_connectivity();
            spiky::SparseShape ss{s, m->max_groups, m->uniform, m->max_row, m->typ_row};
            const int64_t *off = (const int64_t *)m->d_syn_offsets.ptr;
            if (m->uniform) {
                spiky::Scratch scr = m->scratch_fwd.scratch_for(
                    [&](spiky::Scratch &x) { return layout_fill_sparse(m, ss, x); }, "fill_outputs_sparse");
                m->timed("fill_outputs_sparse", st, [&] {
                    check_launch(spiky::launch_fill_sparse_uniform(
                                     ss, weights, lookup_indices, off, (const int64_t *)m->d_in_offsets.ptr,
                                     (const int32_t *)m->d_in_pairs.ptr, (const uint32_t *)m->d_in_order.ptr,
                                     fill_sparse_order_len(m), output, m->int_mode, m->int_rescaler, scr, st),
                                 "fill_outputs_sparse");
                });
            } else {
                m->timed("fill_outputs_sparse", st, [&] {
                    check_hip(spiky::launch_fill_sparse_atomic(ss, weights, lookup_indices, off,
                                                               (const int32_t *)m->d_syn_targets.ptr,
                                                               output, m->int_mode, m->int_rescaler, st),
                              "fill_outputs_sparse");
                });
            }
        }
    });
}

int spiky_lut_forward_step_noalloc(spiky_lut_manager *m, const float *weights,
                                   uint32_t batch_size, const float *input, const int32_t *anchors,
                                   float *output, int32_t *lookup_indices, float cmp_eps,
                                   float *min_deltas, int32_t *min_delta_indices, void *stream) {
    return guarded([&] {
        require_manager(m);
        if (batch_size == 0) throw ValueError("batch_size == 0");
        if (m->sequence_length != 1)
            throw ValueError("forward_step should only be called when sequence_length == 1");
        require_initialized(m);
        if (m->fully_connected != 1)
            throw ValueError("forward_step_noalloc needs a fully connected manager");
        if (!weights || !input || !anchors || !output || !lookup_indices)
            throw ValueError("null tensor pointer");
        if ((min_deltas == nullptr) != (min_delta_indices == nullptr))
            throw ValueError("w_min_anchor_deltas and w_min_anchor_delta_indices must be given together");
        const spiky::FcShape s = m->shape(batch_size);
        const bool tm = spiky::tm_fill_applies(s, m->int_mode);
        const hipStream_t st = as_stream(stream);
        const size_t need =
            tm ? planned_bytes([&](spiky::Scratch &x) { return layout_fill_tm(m, s, x); }, "fill_outputs_fc") : 0;
        if (need > SPIKY_NOALLOC_SCRATCH_BYTES)
            throw ValueError("forward_step_noalloc: this shape needs " + std::to_string(need) +
                             " bytes of scratch, more than the " +
                             std::to_string(SPIKY_NOALLOC_SCRATCH_BYTES) +
                             " the allocation-free path holds; use forward_step");
        m->context_active = true;
        check_hip(spiky::launch_check_detectors(s, input, anchors, cmp_eps, lookup_indices, min_deltas,
                                                min_delta_indices, st),
                  "check_detectors");
        if (!tm) {
            check_hip(spiky::launch_fill_fc_f32(s, weights, lookup_indices, output, m->int_mode,
                                                m->int_rescaler, st),
                      "fill_outputs_fc");
            return;
        }
        // Eager calls on one device are chained through the device's event, so a
        // call on another stream waits for the previous call's kernels to finish
        // with the shared array.  Under stream capture the caller's graph orders
        // its nodes, and an event recorded outside the capture cannot be waited on.
        std::lock_guard<std::mutex> lock(g_noalloc_mutex);
        NoallocDevice &d = noalloc_device();
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        check_hip(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
        const bool eager = cs == hipStreamCaptureStatusNone;
        if (eager && d.recorded) check_hip(hipStreamWaitEvent(st, d.done, 0), "hipStreamWaitEvent(noalloc)");
        spiky::Scratch scr = spiky::scratch_run(d.ptr, SPIKY_NOALLOC_SCRATCH_BYTES);
        check_launch(spiky::launch_fill_tm(s, weights, lookup_indices, output, m->int_mode, m->int_rescaler,
                                           scr, st),
                     "fill_outputs_fc");
        if (eager) {
            check_hip(hipEventRecord(d.done, st), "hipEventRecord(noalloc)");
            d.recorded = true;
        }
    });
}

int spiky_lut_forward_step_i8(spiky_lut_manager *m, const int8_t *q8, const float *scales,
                              uint32_t batch_size, const float *input, const int32_t *anchors,
                              float *output, int32_t *lookup_indices, float cmp_eps,
                              float *min_deltas, int32_t *min_delta_indices, void *stream) {
    return guarded([&] {
        require_manager(m);
        if (batch_size == 0) throw ValueError("batch_size == 0");
        if (m->sequence_length != 1)
            throw ValueError("forward_step should only be called when sequence_length == 1");
        require_initialized(m);
        if (m->fully_connected != 1) throw ValueError("int8 tables need a fully connected manager");
        if (!q8 || !scales || !input || !anchors || !output || !lookup_indices)
            throw ValueError("null tensor pointer");
        if ((min_deltas == nullptr) != (min_delta_indices == nullptr))
            throw ValueError("w_min_anchor_deltas and w_min_anchor_delta_indices must be given together");
        ScopedTimer timer(m->stats, "lut::runtime::forward_non_seq_i8");
        m->context_active = true;
        const hipStream_t st = as_stream(stream);
        const spiky::FcShape s = m->shape(batch_size);
        m->timed("check_detectors", st, [&] {
            check_hip(spiky::launch_check_detectors(s, input, anchors, cmp_eps, lookup_indices,
                                                    min_deltas, min_delta_indices, st),
                      "check_detectors");
        });
        if (spiky::tm_fill_applies(s, m->int_mode)) {
            spiky::Scratch scr = m->scratch_fwd.scratch_for(
                [&](spiky::Scratch &x) { return layout_fill_tm_i8(m, s, x); }, "fill_outputs_fc_i8");
            m->timed("fill_outputs_fc_i8", st, [&] {
                check_launch(spiky::launch_fill_tm_i8(s, q8, scales, lookup_indices, output, m->int_mode,
                                                      m->int_rescaler, scr, st),
                             "fill_outputs_fc_i8");
            });
        } else {
            m->timed("fill_outputs_fc_i8", st, [&] {
                check_hip(spiky::launch_fill_fc_i8(s, q8, scales, lookup_indices, output, m->int_mode,
                                                   m->int_rescaler, st),
                          "fill_outputs_fc_i8");
            });
        }
    });
}

int spiky_lut_backward_backprop(spiky_lut_manager *m, float *weights, uint32_t batch_size,
                                const float *output_grad, const int32_t *anchors,
                                const int32_t *lookup_indices, const float *min_deltas,
                                const int32_t *min_delta_indices, float *input_grad,
                                double external_lr, float *weight_grad,
                                int overwrite_weight_grad, void *stream) {
    return guarded([&] {
        require_manager(m);
        // lut.cu:1044-1049 and lut_runtime.cu:228-238
        if (batch_size == 0) throw ValueError("batch_size == 0");
        if (!m->context_active) throw ValueError("no active context");
        if (m->sequence_length != 1)
            throw ValueError("backward_backprop should only be called when sequence_length == 1");
        require_initialized(m);
        const float ext = (float)external_lr;  // the reference narrows it to fp32 (lut.cu:1082)
        if (ext >= 0.0f && weight_grad != nullptr)
            throw ValueError("in internal weight gradients mode w_weights_gradients should be nullptr");
        if (ext >= 0.0f && m->int_mode)
            throw ValueError("summation dtype torch.int32 can't be combined with GradientType.Internal");
        if (!weights || !output_grad || !anchors || !lookup_indices || !min_deltas ||
            !min_delta_indices || !input_grad)
            throw ValueError("null tensor pointer");
        ScopedTimer timer(m->stats, "lut::runtime::backward_non_seq::backprop");
        const hipStream_t st = as_stream(stream);
        const spiky::FcShape s = m->shape(batch_size);
        // gather_weight_gradients_*: lr = meta lr, times -external_lr in Internal mode (proto:731-734)
        double lr = (double)m->metas[0][0];
        if (ext >= 0.0f) lr *= -(double)ext;
        float *target = (ext >= 0.0f) ? weights : weight_grad;
        const bool overwrite = overwrite_weight_grad != 0 && target == weight_grad;
        if (m->fully_connected == 1) {
            const FcBackwardRegions r = fc_backward_regions(m, s, target != nullptr);
            const bool tm = r.tm;
            uint8_t *base = reinterpret_cast<uint8_t *>(m->scratch.ensure(r.prop_bytes + r.wg_bytes));
            const size_t cap = base ? m->scratch.bytes : 0;
            spiky::Scratch prop_scr = spiky::scratch_run(base, r.prop_bytes);
            spiky::Scratch wg_scr = spiky::scratch_run(base ? base + r.prop_bytes : nullptr, cap - r.prop_bytes);
            m->timed("propagate_fc", st, [&] {
                if (tm)
                    check_launch(spiky::launch_propagate_tm(s, weights, output_grad, lookup_indices,
                                                            min_deltas, min_delta_indices, anchors,
                                                            input_grad, prop_scr, st),
                                 "propagate_through_detectors_fc");
                else
                    check_hip(spiky::launch_propagate_fc(s, weights, output_grad, lookup_indices,
                                                         min_deltas, min_delta_indices, anchors,
                                                         input_grad, m->int_mode, m->int_rescaler, st),
                              "propagate_through_detectors_fc");
            });
            if (m->int_mode)
                check_hip(spiky::launch_convert_i2f(input_grad, (uint64_t)batch_size * m->n_inputs,
                                                    m->int_rescaler, st),
                          "convert_integers_to_floats");
            if (target) {
                m->timed("gather_w_gradients_fc", st, [&] {
                    // the table-major propagate left the transposed keys at its scratch start
                    const uint32_t *key_t = tm ? reinterpret_cast<const uint32_t *>(base) : nullptr;
                    check_launch(spiky::launch_wgrad_fc(s, output_grad, lookup_indices, target, lr,
                                                        m->int_mode, m->int_rescaler, overwrite, wg_scr, st,
                                                        key_t, spiky::tm_key_pitch(s.batch),
                                                        spiky::tm_key_row_shift(s)),
                                 "gather_w_gradients_fc");
                });
            }
        } else {
            m->sync_connectivity();
            spiky::SparseShape ss{s, m->max_groups, m->uniform, m->max_row, m->typ_row};
            const int64_t *off = (const int64_t *)m->d_syn_offsets.ptr;
            const int32_t *tg = (const int32_t *)m->d_syn_targets.ptr;
            m->timed("propagate_sparse", st, [&] {
                check_hip(spiky::launch_propagate_sparse(ss, weights, output_grad, lookup_indices,
                                                         min_deltas, min_delta_indices, anchors, off, tg,
                                                         input_grad, m->int_mode, m->int_rescaler, st),
                          "propagate_through_detectors_sparse");
            });
            if (m->int_mode)
                check_hip(spiky::launch_convert_i2f(input_grad, (uint64_t)batch_size * m->n_inputs,
                                                    m->int_rescaler, st),
                          "convert_integers_to_floats");
            if (target) {
                const uint64_t n_syn = m->syn_targets.size();
                spiky::Scratch scr = m->scratch.scratch_for(
                    [&](spiky::Scratch &x) { return layout_wgrad_sparse(m, ss, x); }, "gather_w_gradients_sparse");
                m->timed("gather_w_gradients_sparse", st, [&] {
                    check_launch(spiky::launch_wgrad_sparse(ss, output_grad, lookup_indices, off, tg,
                                                            (const int32_t *)m->d_syn_neuron.ptr,
                                                            (const int32_t *)m->d_row_pairs.ptr,
                                                            (uint32_t)(m->row_pairs.size() / 2), target, lr,
                                                            overwrite, m->int_mode, m->int_rescaler, scr, n_syn,
                                                            st),
                                 "gather_w_gradients_sparse");
                });
            }
        }
    });
}

static spiky::SeqShape seq_shape(const spiky_lut_manager *m, uint32_t batch) {
    spiky::SeqShape s;
    s.batch = batch;
    s.seq = m->sequence_length;
    s.n_inputs = m->n_inputs;
    s.n_outputs = m->n_outputs;
    s.n_detectors = m->n_detectors;
    s.n_anchors = m->n_anchors;
    s.pe_dim = m->positional_dim;
    s.dgs = m->backward_group_size;
    s.ogs = m->forward_group_size;
    return s;
}

static void require_seq(const spiky_lut_manager *m, uint32_t batch_size, const char *what) {
    if (batch_size == 0) throw ValueError("batch_size == 0");
    // lut_runtime.cu:438-440 / 620-622
    if (m->sequence_length <= 1)
        throw ValueError(std::string(what) + " should only be called when sequence_length > 1");
    require_initialized(m);
    if (2 * m->n_anchors + m->positional_dim > 24)
        throw ValueError("2 * n_anchors_per_detector + positional_dim > 24 is not supported");
    if ((uint64_t)batch_size * m->sequence_length > 0x7fffffffull)
        throw ValueError("batch_size * sequence_length is too large");
}

int spiky_lut_forward_step_concat(spiky_lut_manager *m, const float *weights, uint32_t batch_size,
                                  const float *input, const int32_t *anchors, float *output,
                                  int32_t *lookup_indices, float cmp_eps,
                                  const float *positional_embeddings,
                                  int32_t *positional_lookup_indices, float *min_deltas,
                                  int32_t *min_delta_indices, float *positional_min_deltas,
                                  int32_t *positional_min_delta_indices, void *stream) {
    return guarded([&] {
        require_manager(m);
        require_seq(m, batch_size, "forward_step_concat");
        if (!weights || !input || !anchors || !output || !lookup_indices)
            throw ValueError("null tensor pointer");
        const bool train = min_deltas != nullptr;
        if ((min_delta_indices != nullptr) != train)
            throw ValueError("w_min_anchor_deltas and w_min_anchor_delta_indices must be given together");
        if (m->positional_dim > 0) {
            // lut.cu:737-777
            if (!positional_embeddings) throw ValueError("r_positional_embeddings must be provided when positional_dim > 0");
            if (!positional_lookup_indices) throw ValueError("w_positional_lookup_indices must be provided when positional_dim > 0");
            if (train && (!positional_min_deltas || !positional_min_delta_indices))
                throw ValueError("positional min deltas must be provided in training mode when positional_dim > 0");
        }
        ScopedTimer timer(m->stats, train ? "lut::runtime::forward_seq" : "lut::runtime::forward_seq_eval");
        m->context_active = true;
        const hipStream_t st = as_stream(stream);
        const spiky::SeqShape s = seq_shape(m, batch_size);
        if (m->fully_connected != 1) {
            // sparse lookup connectivity (lut_runtime.cu:518-545)
            m->sync_connectivity();
            if (!spiky::seq_sparse_applies(s, m->max_groups))
                throw ValueError("sequence shape too large for the sparse sequence path");
            m->timed("check_detectors_seq", st, [&] {
                check_hip(spiky::launch_seq_indices(s, input, anchors, positional_embeddings,
                                                    lookup_indices, positional_lookup_indices,
                                                    min_deltas, min_delta_indices,
                                                    positional_min_deltas,
                                                    positional_min_delta_indices, cmp_eps, st),
                          "check_detectors_seq");
            });
            m->timed("fill_outputs_sparse_seq", st, [&] {
                check_hip(spiky::launch_fill_seq_sparse(s, m->max_groups, weights, lookup_indices,
                                                        positional_lookup_indices,
                                                        (const int64_t *)m->d_syn_offsets.ptr,
                                                        (const int32_t *)m->d_syn_targets.ptr, output,
                                                        m->int_mode, m->int_rescaler, st),
                          "forward_step_concat");
            });
            return;
        }
        spiky::Scratch scr = m->scratch_fwd.scratch_for(
            [&](spiky::Scratch &x) { return layout_forward_seq(m, s, x); }, "forward_step_concat");
        m->timed("fill_outputs_seq", st, [&] {
            check_launch(spiky::launch_forward_seq(s, weights, input, anchors, positional_embeddings,
                                                output, lookup_indices, positional_lookup_indices,
                                                min_deltas, min_delta_indices, positional_min_deltas,
                                                positional_min_delta_indices, cmp_eps, m->int_mode,
                                                m->int_rescaler, scr, st),
                      "forward_step_concat");
        });
    });
}

int spiky_lut_backward_backprop_concat(spiky_lut_manager *m, float *weights, uint32_t batch_size,
                                       const float *output_grad, const int32_t *anchors,
                                       const int32_t *lookup_indices, const float *min_deltas,
                                       const int32_t *min_delta_indices, float *input_grad,
                                       double external_lr, const int32_t *positional_lookup_indices,
                                       const float *positional_min_deltas,
                                       const int32_t *positional_min_delta_indices,
                                       float *positional_grad, float *weight_grad,
                                       int overwrite_weight_grad, void *stream) {
    return guarded([&] {
        require_manager(m);
        if (batch_size == 0) throw ValueError("batch_size == 0");
        if (!m->context_active) throw ValueError("no active context");
        require_seq(m, batch_size, "backward_backprop_concat");
        const float ext = (float)external_lr;
        if (ext >= 0.0f && weight_grad != nullptr)
            throw ValueError("in internal weight gradients mode w_weights_gradients should be nullptr");
        if (ext >= 0.0f && m->int_mode)
            throw ValueError("summation dtype torch.int32 can't be combined with GradientType.Internal");
        if (!weights || !output_grad || !anchors || !lookup_indices || !min_deltas ||
            !min_delta_indices || !input_grad)
            throw ValueError("null tensor pointer");
        if (m->positional_dim > 0 && (!positional_lookup_indices || !positional_min_deltas ||
                                      !positional_min_delta_indices || !positional_grad))
            throw ValueError("positional tensors must be provided when positional_dim > 0");
        ScopedTimer timer(m->stats, "lut::runtime::backward_seq");
        const hipStream_t st = as_stream(stream);
        const spiky::SeqShape s = seq_shape(m, batch_size);
        double lr = (double)m->metas[0][0];
        if (ext >= 0.0f) lr *= -(double)ext;
        float *target = (ext >= 0.0f) ? weights : weight_grad;
        const bool overwrite = overwrite_weight_grad != 0 && target == weight_grad;
        if (m->fully_connected != 1) {
            // sparse lookup connectivity (lut_runtime.cu:639-740)
            m->sync_connectivity();
            if (!spiky::seq_sparse_applies(s, m->max_groups))
                throw ValueError("sequence shape too large for the sparse sequence path");
            m->timed("backward_seq_sparse", st, [&] {
                check_hip(spiky::launch_backward_seq_sparse(
                              s, m->max_groups, weights, output_grad, anchors, lookup_indices,
                              min_deltas, min_delta_indices, positional_lookup_indices,
                              positional_min_deltas, positional_min_delta_indices,
                              (const int64_t *)m->d_syn_offsets.ptr,
                              (const int32_t *)m->d_syn_targets.ptr, m->syn_targets.size(),
                              input_grad, positional_grad, target, lr, overwrite, m->int_mode,
                              m->int_rescaler, st),
                          "backward_backprop_concat");
            });
            return;
        }
        spiky::Scratch scr = m->scratch.scratch_for(
            [&](spiky::Scratch &x) { return layout_backward_seq(m, s, x); }, "backward_backprop_concat");
        m->timed("backward_seq", st, [&] {
            check_launch(spiky::launch_backward_seq(s, weights, output_grad, anchors, lookup_indices,
                                                 min_deltas, min_delta_indices,
                                                 positional_lookup_indices, positional_min_deltas,
                                                 positional_min_delta_indices, input_grad,
                                                 positional_grad, target, lr, overwrite, m->int_mode,
                                                 m->int_rescaler, scr, st),
                      "backward_backprop_concat");
        });
    });
}

// Product mode: the manager is built with sequence_length 1 and n_inputs
// 2 * n + pd; the real sequence length comes with each call (lut.cu:880-887).
static spiky::ProductShape product_shape(const spiky_lut_manager *m, uint32_t batch_size,
                                         uint32_t sequence_length, uint32_t n_inputs_1,
                                         uint32_t n_inputs_2, int sliced_mode, float cmp_eps,
                                         const char *what) {
    if (batch_size == 0) throw ValueError("batch_size == 0");
    if (m->sequence_length != 1)
        throw ValueError(std::string(what) +
                         ": this is an experimental method, this->sequence_length should be equal to "
                         "1, real length of the sequence is passed as the method parameter");
    if (sequence_length == 0) throw ValueError("sequence_length == 0");
    require_initialized(m);
    spiky::ProductShape s;
    s.batch = batch_size;
    s.seq_len = sequence_length;
    s.n1 = n_inputs_1;
    s.n2 = n_inputs_2;
    s.pd = m->positional_dim;
    s.n_detectors = m->n_detectors;
    s.n_anchors = m->n_anchors;
    s.n_outputs = m->n_outputs;
    s.sliced = sliced_mode != 0;
    s.cmp_eps = cmp_eps;
    if (m->fully_connected == 1 && !spiky::product_applies(s))
        throw ValueError("product mode shape out of range (n_detectors * 2^n_anchors must be <= 16384, "
                         "batch_size * sequence_length <= 4194240)");
    if (m->fully_connected != 1 && !spiky::product_sparse_applies(s))
        throw ValueError("product mode shape out of range for sparse connectivity");
    return s;
}

int spiky_lut_forward_step_product(spiky_lut_manager *m, const float *weights, uint32_t batch_size,
                                   uint32_t sequence_length, const float *input_1,
                                   const float *input_2, const int32_t *anchors, float *output,
                                   uint32_t n_inputs_1, uint32_t n_inputs_2, int sliced_mode,
                                   float cmp_eps, const float *positional_embeddings,
                                   void *stream) {
    return guarded([&] {
        require_manager(m);
        const spiky::ProductShape s = product_shape(m, batch_size, sequence_length, n_inputs_1,
                                                    n_inputs_2, sliced_mode, cmp_eps,
                                                    "forward_step_product");
        if (!weights || !input_1 || !input_2 || !anchors || !output)
            throw ValueError("null tensor pointer");
        if (s.pd > 0 && !positional_embeddings)
            throw ValueError("r_positional_embeddings must be provided when positional_dim > 0");
        ScopedTimer timer(m->stats, "lut::runtime::forward_product");
        m->context_active = true;
        const hipStream_t st = as_stream(stream);
        if (m->fully_connected == 1) {
            spiky::Scratch scr = m->scratch_fwd.scratch_for(
                [&](spiky::Scratch &x) { return layout_forward_product(m, s, x); }, "forward_step_product");
            m->timed("fill_outputs_product", st, [&] {
                check_launch(spiky::launch_forward_product(s, weights, input_1, input_2,
                                                        positional_embeddings, anchors, output,
                                                        m->int_mode, m->int_rescaler, scr, st),
                          "forward_step_product");
            });
        } else {
            m->sync_connectivity();
            m->timed("fill_outputs_product_sparse", st, [&] {
                check_hip(spiky::launch_forward_product_sparse(
                              s, weights, input_1, input_2, positional_embeddings, anchors,
                              (const int64_t *)m->d_syn_offsets.ptr,
                              (const int32_t *)m->d_syn_targets.ptr, output, m->int_mode,
                              m->int_rescaler, st),
                          "forward_step_product");
            });
        }
        if (m->int_mode)
            check_hip(spiky::launch_convert_i2f(output, (uint64_t)s.batch * s.seq_len * s.n_outputs,
                                                m->int_rescaler, st),
                      "convert_integers_to_floats");
    });
}

int spiky_lut_backward_backprop_product(spiky_lut_manager *m, float *weights, uint32_t batch_size,
                                        uint32_t sequence_length, const float *input_1,
                                        const float *input_2, const int32_t *anchors,
                                        const float *output_grad, float *input_grad_1,
                                        float *input_grad_2, double external_lr,
                                        uint32_t n_inputs_1, uint32_t n_inputs_2, int sliced_mode,
                                        float cmp_eps, float *weight_grad,
                                        const float *positional_embeddings, float *positional_grad,
                                        void *stream) {
    return guarded([&] {
        require_manager(m);
        if (batch_size == 0) throw ValueError("batch_size == 0");
        if (!m->context_active) throw ValueError("no active context");
        const spiky::ProductShape s = product_shape(m, batch_size, sequence_length, n_inputs_1,
                                                    n_inputs_2, sliced_mode, cmp_eps,
                                                    "backward_backprop_product");
        // lut_runtime.cu:1075-1077
        if (external_lr >= 0.0 && weight_grad != nullptr)
            throw ValueError("in internal weight gradients mode w_weights_gradients should be nullptr");
        if (external_lr >= 0.0 && m->int_mode)
            throw ValueError("summation dtype torch.int32 can't be combined with GradientType.Internal");
        if (!weights || !input_1 || !input_2 || !anchors || !output_grad || !input_grad_1 ||
            !input_grad_2)
            throw ValueError("null tensor pointer");
        if (s.pd > 0 && (!positional_embeddings || !positional_grad))
            throw ValueError("positional embeddings and their gradients must be provided when positional_dim > 0");
        ScopedTimer timer(m->stats, "lut::runtime::backward_product");
        const hipStream_t st = as_stream(stream);
        double lr = (double)m->metas[0][0];
        if (external_lr >= 0.0) lr *= -external_lr;
        float *target = (external_lr >= 0.0) ? weights : weight_grad;
        if (m->fully_connected == 1) {
            spiky::Scratch scr = m->scratch.scratch_for(
                [&](spiky::Scratch &x) { return layout_backward_product(m, s, x); }, "backward_backprop_product");
            m->timed("backward_product", st, [&] {
                check_launch(spiky::launch_backward_product(s, weights, input_1, input_2,
                                                         positional_embeddings, anchors, output_grad,
                                                         input_grad_1, input_grad_2, positional_grad,
                                                         target, lr, m->int_mode, m->int_rescaler, scr,
                                                         st),
                          "backward_backprop_product");
            });
        } else {
            m->sync_connectivity();
            m->timed("backward_product_sparse", st, [&] {
                check_hip(spiky::launch_backward_product_sparse(
                              s, weights, input_1, input_2, positional_embeddings, anchors,
                              (const int64_t *)m->d_syn_offsets.ptr,
                              (const int32_t *)m->d_syn_targets.ptr, output_grad, input_grad_1,
                              input_grad_2, positional_grad, target, lr, m->int_mode,
                              m->int_rescaler, st),
                          "backward_backprop_product");
            });
        }
        if (m->int_mode) {
            // lut_runtime.cu:1405-1456: every buffer this call summed into
            const uint64_t bs = (uint64_t)s.batch * s.seq_len;
            check_hip(spiky::launch_convert_i2f(input_grad_1, bs * s.n1, m->int_rescaler, st),
                      "convert_integers_to_floats");
            if (input_grad_2 != input_grad_1)
                check_hip(spiky::launch_convert_i2f(input_grad_2, bs * s.n2, m->int_rescaler, st),
                          "convert_integers_to_floats");
            if (weight_grad)
                check_hip(spiky::launch_convert_i2f(weight_grad, spiky_lut_weights_dimension(m),
                                                    m->int_rescaler, st),
                          "convert_integers_to_floats");
            if (s.pd > 0)
                check_hip(spiky::launch_convert_i2f(
                              positional_grad, (uint64_t)s.pd * s.n_detectors * (s.seq_len - 1),
                              m->int_rescaler, st),
                          "convert_integers_to_floats");
        }
    });
}

int spiky_lut_decode_anchors_compact(const uint32_t *encoded_pairs, uint32_t n_detectors,
                                     uint32_t max_pairs_per_detector, uint32_t n_anchors,
                                     const int64_t *in_offsets, const int32_t *in_ids,
                                     int32_t *anchors_out) {
    return guarded([&] {
        if (!encoded_pairs || !in_offsets || !anchors_out) throw ValueError("null pointer");
        if (max_pairs_per_detector < n_anchors)
            throw ValueError("max_pairs_per_detector < n_anchors_per_detector");
        // lut_compile_time_kernels_logic.proto:70-125 (compact decode); lut.cu:537-550 (error)
        uint64_t errors = 0;
        for (uint32_t i = 0; i < n_detectors; i++) {
            const uint32_t *codes = encoded_pairs + (size_t)i * max_pairs_per_detector;
            const int64_t len = in_offsets[i + 1] - in_offsets[i];
            if (len <= 1) { errors++; continue; }
            const uint32_t n_syn = (uint32_t)len;
            const uint32_t max_codes = n_syn * (n_syn - 1);
            const int32_t *ids = in_ids + in_offsets[i];
            int32_t *dst = anchors_out + (size_t)i * n_anchors * 2;
            for (uint32_t j = 0; j < n_anchors; j++) {
                const uint32_t c = codes[j] % max_codes;
                uint32_t a1 = c / (n_syn - 1);
                uint32_t a2 = c % (n_syn - 1);
                if (a2 >= a1) a2++;
                dst[2 * j] = ids[a1];
                dst[2 * j + 1] = ids[a2];
            }
        }
        if (errors) throw ValueError("Some detectors have <= 1 input synapses");
    });
}

// ---- dense -> sparse converter (torch_utils.cu:11-339) ---------------------

uint64_t spiky_densify32_workspace_bytes(uint64_t n) { return spiky::densify32_workspace_bytes(n); }

int spiky_count_nonzero32(const void *source, uint64_t n, void *workspace,
                          uint64_t workspace_bytes, int64_t *counter, void *stream) {
    return guarded([&] {
        // torch_utils.py:63-67 (the size rule; the dtype rule is the caller's)
        if (n % 4 != 0) throw ValueError("source tensor size must be divisable by 4");
        if (!counter || (n > 0 && !source)) throw ValueError("null pointer");
        if (!workspace || workspace_bytes < spiky::densify32_workspace_bytes(n))
            throw ValueError("densify workspace too small");
        check_hip(spiky::launch_densify32_count(static_cast<const uint32_t *>(source), n, workspace,
                                                counter, as_stream(stream)),
                  "count_nonzero");
    });
}

int spiky_dense_to_sparse32(void *source, uint64_t n, int64_t *indices, void *values,
                            uint64_t capacity, void *workspace, uint64_t workspace_bytes,
                            int64_t *counter, int erase_input, int counted, void *stream) {
    return guarded([&] {
        if (n % 4 != 0) throw ValueError("source tensor size must be divisable by 4");
        if (!counter || (n > 0 && !source) || (capacity > 0 && (!indices || !values)))
            throw ValueError("null pointer");
        if (!workspace || workspace_bytes < spiky::densify32_workspace_bytes(n))
            throw ValueError("densify workspace too small");
        const hipStream_t st = as_stream(stream);
        uint32_t *src = static_cast<uint32_t *>(source);
        if (!counted)
            check_hip(spiky::launch_densify32_count(src, n, workspace, counter, st), "dense_to_sparse_32");
        check_hip(spiky::launch_densify32_write(src, n, workspace, indices,
                                                static_cast<uint32_t *>(values), capacity,
                                                erase_input != 0, st),
                  "dense_to_sparse_32");
    });
}

int spiky_lut_profiling_stats(const spiky_lut_manager *m, char *buf, uint64_t buf_len) {
    return guarded([&] {
        require_manager(m);
        std::string s;
        for (const auto &kv : m->stats) {
            char line[256];
            std::snprintf(line, sizeof(line), "%s: %.3f ms / %llu = %.3f ms\n", kv.first.c_str(),
                          kv.second.total_ms, (unsigned long long)kv.second.count,
                          kv.second.count ? kv.second.total_ms / kv.second.count : 0.0);
            s += line;
        }
        if (buf && buf_len) {
            std::strncpy(buf, s.c_str(), buf_len - 1);
            buf[buf_len - 1] = 0;
        }
    });
}

void spiky_lut_reset_profiler(spiky_lut_manager *m) {
    if (m) m->stats.clear();
}

int spiky_lut_scratch_plan(spiky_lut_manager *m, int op, uint32_t batch_size, uint32_t sequence_length,
                           uint32_t n_inputs_1, uint32_t n_inputs_2, int sliced_mode, uint64_t capacity,
                           uint64_t *needed) {
    return guarded([&] {
        require_manager(m);
        if (!needed) throw ValueError("null output pointer");
        *needed = 0;
        if (batch_size == 0) throw ValueError("batch_size == 0");
        require_initialized(m);
        const bool fc = m->fully_connected == 1;
        // a launcher's layout checked against its region [offset, capacity) of
        // the entry point's buffer (Check mode launches nothing)
        auto check_region = [&](auto &&layout, uint64_t offset, uint64_t region, const char *what) {
            spiky::Scratch x;
            x.mode = spiky::Scratch::Check;
            x.bytes = capacity > offset ? std::min<uint64_t>(capacity - offset, region) : 0;
            if (layout(x) != hipSuccess) {
                std::string why = spiky::scratch_refusal();
                spiky::scratch_refusal().clear();
                throw ValueError(why.empty() ? std::string(what) + ": layout refused" : why);
            }
        };
        auto single = [&](auto &&layout, const char *what) {
            *needed = planned_bytes(layout, what);
            check_region(layout, 0, UINT64_MAX, what);
        };
        switch (op) {
            case SPIKY_OP_FORWARD:
            case SPIKY_OP_FORWARD_I8: {
                if (m->sequence_length != 1)
                    throw ValueError("forward_step should only be called when sequence_length == 1");
                if (op == SPIKY_OP_FORWARD_I8 && !fc) throw ValueError("int8 tables need a fully connected manager");
                const spiky::FcShape s = m->shape(batch_size);
                if (fc && spiky::tm_fill_applies(s, m->int_mode)) {
                    if (op == SPIKY_OP_FORWARD)
                        single([&](spiky::Scratch &x) { return layout_fill_tm(m, s, x); }, "fill_outputs_fc");
                    else
                        single([&](spiky::Scratch &x) { return layout_fill_tm_i8(m, s, x); }, "fill_outputs_fc_i8");
                } else if (!fc && m->uniform) {
                    const spiky::SparseShape ss{s, m->max_groups, m->uniform, m->max_row, m->typ_row};
                    single([&](spiky::Scratch &x) { return layout_fill_sparse(m, ss, x); }, "fill_outputs_sparse");
                }
                break;
            }
            case SPIKY_OP_BACKWARD:
            case SPIKY_OP_BACKWARD_NO_WGRAD: {
                if (m->sequence_length != 1)
                    throw ValueError("backward_backprop should only be called when sequence_length == 1");
                const bool wg = op == SPIKY_OP_BACKWARD;
                const spiky::FcShape s = m->shape(batch_size);
                if (fc) {
                    const FcBackwardRegions r = fc_backward_regions(m, s, wg);
                    *needed = r.prop_bytes + r.wg_bytes;
                    if (r.tm)
                        check_region([&](spiky::Scratch &x) { return layout_propagate_tm(s, x); }, 0, r.prop_bytes,
                                     "propagate_through_detectors_fc");
                    if (wg)
                        check_region([&](spiky::Scratch &x) { return layout_wgrad_fc(m, s, x); }, r.prop_bytes,
                                     UINT64_MAX, "gather_w_gradients_fc");
                } else if (wg) {
                    const spiky::SparseShape ss{s, m->max_groups, m->uniform, m->max_row, m->typ_row};
                    single([&](spiky::Scratch &x) { return layout_wgrad_sparse(m, ss, x); },
                           "gather_w_gradients_sparse");
                }
                break;
            }
            case SPIKY_OP_FORWARD_CONCAT:
            case SPIKY_OP_BACKWARD_CONCAT: {
                const bool fwd = op == SPIKY_OP_FORWARD_CONCAT;
                require_seq(m, batch_size, fwd ? "forward_step_concat" : "backward_backprop_concat");
                const spiky::SeqShape s = seq_shape(m, batch_size);
                if (fc) {
                    if (fwd)
                        single([&](spiky::Scratch &x) { return layout_forward_seq(m, s, x); }, "forward_step_concat");
                    else
                        single([&](spiky::Scratch &x) { return layout_backward_seq(m, s, x); },
                               "backward_backprop_concat");
                }
                break;
            }
            case SPIKY_OP_FORWARD_PRODUCT:
            case SPIKY_OP_BACKWARD_PRODUCT: {
                const bool fwd = op == SPIKY_OP_FORWARD_PRODUCT;
                const spiky::ProductShape s =
                    product_shape(m, batch_size, sequence_length, n_inputs_1, n_inputs_2, sliced_mode, 0.0f,
                                  fwd ? "forward_step_product" : "backward_backprop_product");
                if (fc) {
                    if (fwd)
                        single([&](spiky::Scratch &x) { return layout_forward_product(m, s, x); },
                               "forward_step_product");
                    else
                        single([&](spiky::Scratch &x) { return layout_backward_product(m, s, x); },
                               "backward_backprop_product");
                }
                break;
            }
            default:
                throw ValueError("unknown operation code " + std::to_string(op));
        }
    });
}

int spiky_lut_set_kernel_timing(spiky_lut_manager *m, int enable) {
    return guarded([&] {
        require_manager(m);
        m->collect();
        m->timing = enable != 0;
    });
}

int spiky_lut_kernel_times(spiky_lut_manager *m, char *buf, uint64_t buf_len, int reset) {
    return guarded([&] {
        require_manager(m);
        m->collect();
        std::string s;
        for (const auto &kv : m->kernel_stats) {
            char line[256];
            std::snprintf(line, sizeof(line), "%s %llu %.6f\n", kv.first.c_str(),
                          (unsigned long long)kv.second.count, kv.second.total_ms);
            s += line;
        }
        if (buf && buf_len) {
            std::strncpy(buf, s.c_str(), buf_len - 1);
            buf[buf_len - 1] = 0;
        }
        if (reset) m->kernel_stats.clear();
    });
}

}  // extern "C"

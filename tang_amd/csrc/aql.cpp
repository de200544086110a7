// Replay of recorded kernel sequences on an HSA queue of the library's own.
//
// A HIP graph or stream launch puts agent-scope fences on every kernel
// dispatch: the command processor writes back the L2 of every XCD after each
// kernel and invalidates it before the next.  Measured on MI355X with
// kernargs in device memory: 1.74 us per dependent dispatch of a small
// kernel with those fences (the same as a HIP graph node, 1.79) against 1.30
// with none, and 5.76 against 5.24 us for a chain of 24 MB reads.  The decode
// step and the benchmarked GEMV chain are sequences of small dependent
// kernels, so this file dispatches them itself: each recorded kernel becomes
// an AQL packet whose kernarg segment sits in device memory, the packets of
// a sequence carry no release fences between them (only the acquire), the
// first acquires and the last releases at system scope.  Without the
// release, data a kernel leaves in its XCD's L2 is not visible to the next
// kernel on another XCD, so every kernel of such a sequence writes the
// values a later kernel reads with write-through stores (st_coherent,
// relaxed agent-scope atomic stores).
// The library records a sequence as write-through only when all its
// kernels are; any other sequence keeps agent-scope fences.
//
// The kernels come from the library's own code objects: the gfx950 entries
// of the clang offload bundles in the .hip_fatbin section of this shared
// object, loaded into HSA executables.  A launch names its kernel by the
// host-side handle HIP uses; dladdr gives the handle's symbol, which is the
// kernel's mangled name, and the executables hold the kernel descriptor
// under that name plus ".kd".  Kernels that use __device__ globals must not
// be recorded: the executables hold their own copies of such variables.
#include <dlfcn.h>
#include <elf.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <functional>
#include <iterator>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "aql.hpp"
#include "capi_util.hpp"

namespace th {

namespace {

#define TH_HSA(expr)                                                                                \
    do {                                                                                            \
        hsa_status_t s_ = (expr);                                                                   \
        if (s_ != HSA_STATUS_SUCCESS) {                                                             \
            const char* m_ = nullptr;                                                               \
            hsa_status_string(s_, &m_);                                                             \
            throw Error(TH_ERR_HIP, std::string(#expr) + ": " + (m_ ? m_ : "HSA error"));           \
        }                                                                                           \
    } while (0)

constexpr uint32_t QUEUE_PACKETS = 4096;
constexpr size_t KERNARG_ALIGN = 64;
constexpr size_t HIDDEN_ARGS_BYTES = 256;  // code object v5 implicit arguments
constexpr double WAIT_LIMIT_S = 120.0;

struct KernelInfo {
    uint64_t object = 0;
    uint32_t kernarg_bytes = 0, group_bytes = 0, private_bytes = 0;
    bool write_through = false;  // listed in WRITE_THROUGH_KERNELS
};

// The kernels a write-through sequence may hold: every global store they make
// is write-through (relaxed agent-scope atomic stores, `sc1`), so no release
// fence is needed between them and the kernels after them.  An entry matches
// a mangled kernel name that contains both strings (epilogue "" = any).
// tests/test_aql_write_through.py disassembles the built library and checks
// every store of every kernel an entry matches; aql_record_launch refuses a
// kernel no entry matches in a write-through sequence.
struct WriteThroughKernel {
    const char* kernel;
    const char* epilogue;
};
const WriteThroughKernel WRITE_THROUGH_KERNELS[] = {
    {"q4_gemv_kernel", "EpiStore"},
    {"q4_gemv_kernel", "EpiQKV"},
    {"q4_gemv_kernel", "EpiAddToSsq"},
    {"q4_gemv_kernel", "EpiSwiGLU"},
    {"q4_gemv_kernel", "EpiTileMax"},
    {"q8_gemv_kernel", "EpiStore"},
    {"attn_decode_kernel", ""},
    {"llama_argmax_embed_kernel", ""},
    {"aql_stamp_kernel", ""},
};

bool is_write_through_kernel(const std::string& mangled) {
    for (const WriteThroughKernel& w : WRITE_THROUGH_KERNELS)
        if (mangled.find(w.kernel) != std::string::npos && mangled.find(w.epilogue) != std::string::npos) return true;
    return false;
}

// Per-process: the code objects of this library, loaded once per agent.
struct Program {
    hsa_agent_t agent{};
    // the code object images stay alive with the executables: the loader
    // reports their memory as the loaded code objects' storage
    // (hsa_ven_amd_loader), so it must stay valid
    std::vector<std::string> images;
    std::vector<hsa_executable_t> exes;
    std::unordered_map<std::string, KernelInfo> by_name;
    std::unordered_map<const void*, KernelInfo> by_handle;
};

thread_local AqlSeq* g_recording = nullptr;
std::mutex g_mu;
std::vector<Program*> g_programs;

hsa_status_t collect_gpu(hsa_agent_t a, void* data) {
    hsa_device_type_t t;
    if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) == HSA_STATUS_SUCCESS && t == HSA_DEVICE_TYPE_GPU)
        ((std::vector<hsa_agent_t>*)data)->push_back(a);
    return HSA_STATUS_SUCCESS;
}

// The HSA agent of HIP device `ordinal` (same PCI location).
hsa_agent_t agent_of(int ordinal) {
    std::vector<hsa_agent_t> gpus;
    TH_HSA(hsa_iterate_agents(collect_gpu, &gpus));
    TH_REQUIRE(!gpus.empty(), "no HSA GPU agent");
    int bus = -1, dev = -1, dom = -1;
    TH_HIP(hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, ordinal));
    TH_HIP(hipDeviceGetAttribute(&dev, hipDeviceAttributePciDeviceId, ordinal));
    TH_HIP(hipDeviceGetAttribute(&dom, hipDeviceAttributePciDomainID, ordinal));
    for (hsa_agent_t a : gpus) {
        uint32_t bdf = 0, domain = 0;
        if (hsa_agent_get_info(a, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_BDFID, &bdf) != HSA_STATUS_SUCCESS) continue;
        (void)hsa_agent_get_info(a, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_DOMAIN, &domain);
        if ((int)(bdf >> 8) == bus && (int)((bdf >> 3) & 31) == dev && (int)domain == dom) return a;
    }
    TH_REQUIRE(gpus.size() == 1, "no HSA agent matches the HIP device's PCI location");
    return gpus[0];
}

// gfx950 code objects of this shared object's .hip_fatbin section.
std::vector<std::string> own_code_objects() {
    Dl_info di{};
    TH_REQUIRE(dladdr((const void*)&own_code_objects, &di) && di.dli_fname, "cannot locate the library file");
    std::ifstream f(di.dli_fname, std::ios::binary);
    TH_REQUIRE(f.good(), std::string("cannot read ") + di.dli_fname);
    const std::string file((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    TH_REQUIRE(file.size() > sizeof(Elf64_Ehdr), "library file too short");
    Elf64_Ehdr eh;
    std::memcpy(&eh, file.data(), sizeof eh);
    TH_REQUIRE(std::memcmp(eh.e_ident, ELFMAG, SELFMAG) == 0 && eh.e_shoff + (size_t)eh.e_shnum * sizeof(Elf64_Shdr) <= file.size(),
               "library is not a readable ELF64 file");
    std::vector<Elf64_Shdr> sh(eh.e_shnum);
    std::memcpy(sh.data(), file.data() + eh.e_shoff, sh.size() * sizeof(Elf64_Shdr));
    TH_REQUIRE(eh.e_shstrndx < sh.size(), "bad section name table");
    const Elf64_Shdr& names = sh[eh.e_shstrndx];
    std::string fatbin;
    for (const Elf64_Shdr& s : sh) {
        if (s.sh_name >= names.sh_size) continue;
        if (std::strcmp(file.data() + names.sh_offset + s.sh_name, ".hip_fatbin") == 0) {
            TH_REQUIRE(s.sh_offset + s.sh_size <= file.size(), "truncated .hip_fatbin");
            fatbin.assign(file.data() + s.sh_offset, s.sh_size);
        }
    }
    TH_REQUIRE(!fatbin.empty(), "no .hip_fatbin section in the library");
    // clang offload bundles, one per translation unit: magic, entry count,
    // then (offset, size, triple length, triple) per entry.
    static const char MAGIC[] = "__CLANG_OFFLOAD_BUNDLE__";
    const size_t ml = sizeof(MAGIC) - 1;
    std::vector<std::string> out;
    for (size_t at = fatbin.find(MAGIC); at != std::string::npos; at = fatbin.find(MAGIC, at + ml)) {
        size_t p = at + ml;
        auto u64 = [&](size_t& q) {
            TH_REQUIRE(q + 8 <= fatbin.size(), "truncated offload bundle");
            uint64_t v;
            std::memcpy(&v, fatbin.data() + q, 8);
            q += 8;
            return v;
        };
        const uint64_t n = u64(p);
        for (uint64_t e = 0; e < n; e++) {
            const uint64_t off = u64(p), size = u64(p), tl = u64(p);
            TH_REQUIRE(p + tl <= fatbin.size(), "truncated bundle triple");
            const std::string triple(fatbin.data() + p, tl);
            p += tl;
            if (size && triple.find("amdgcn-amd-amdhsa") != std::string::npos && triple.find("gfx950") != std::string::npos) {
                TH_REQUIRE(at + off + size <= fatbin.size(), "truncated code object");
                out.emplace_back(fatbin.data() + at + off, size);
            }
        }
    }
    TH_REQUIRE(!out.empty(), "no gfx950 code object in the library");
    return out;
}

struct SymCtx {
    Program* prog;
};

hsa_status_t collect_kernel(hsa_executable_t, hsa_agent_t, hsa_executable_symbol_t s, void* data) {
    hsa_symbol_kind_t kind;
    if (hsa_executable_symbol_get_info(s, HSA_EXECUTABLE_SYMBOL_INFO_TYPE, &kind) != HSA_STATUS_SUCCESS ||
        kind != HSA_SYMBOL_KIND_KERNEL)
        return HSA_STATUS_SUCCESS;
    uint32_t len = 0;
    (void)hsa_executable_symbol_get_info(s, HSA_EXECUTABLE_SYMBOL_INFO_NAME_LENGTH, &len);
    std::string name(len, '\0');
    (void)hsa_executable_symbol_get_info(s, HSA_EXECUTABLE_SYMBOL_INFO_NAME, name.data());
    if (name.size() > 3 && name.compare(name.size() - 3, 3, ".kd") == 0) name.resize(name.size() - 3);
    KernelInfo k;
    (void)hsa_executable_symbol_get_info(s, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, &k.object);
    (void)hsa_executable_symbol_get_info(s, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE, &k.kernarg_bytes);
    (void)hsa_executable_symbol_get_info(s, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE, &k.group_bytes);
    (void)hsa_executable_symbol_get_info(s, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE, &k.private_bytes);
    k.write_through = is_write_through_kernel(name);
    ((SymCtx*)data)->prog->by_name.emplace(name, k);
    return HSA_STATUS_SUCCESS;
}

Program* program_for(hsa_agent_t agent) {
    for (Program* p : g_programs)
        if (p->agent.handle == agent.handle) return p;
    Program* p = new Program;
    p->agent = agent;
    p->images = own_code_objects();
    for (const std::string& co : p->images) {
        hsa_code_object_reader_t rd;
        TH_HSA(hsa_code_object_reader_create_from_memory(co.data(), co.size(), &rd));
        hsa_executable_t ex;
        TH_HSA(hsa_executable_create_alt(HSA_PROFILE_FULL, HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT, nullptr, &ex));
        TH_HSA(hsa_executable_load_agent_code_object(ex, agent, rd, nullptr, nullptr));
        TH_HSA(hsa_executable_freeze(ex, nullptr));
        (void)hsa_code_object_reader_destroy(rd);
        p->exes.push_back(ex);
        SymCtx ctx{p};
        TH_HSA(hsa_executable_iterate_agent_symbols(ex, agent, collect_kernel, &ctx));
    }
    g_programs.push_back(p);
    return p;
}

// Under g_mu (recordings on several threads share the per-agent cache).
KernelInfo kernel_info(Program* p, const void* handle) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = p->by_handle.find(handle);
    if (it != p->by_handle.end()) return it->second;
    Dl_info di{};
    TH_REQUIRE(dladdr(handle, &di) && di.dli_sname && di.dli_saddr == handle,
               "kernel handle has no exported symbol");
    auto k = p->by_name.find(di.dli_sname);
    TH_REQUIRE(k != p->by_name.end(), std::string("kernel not in the library's code objects: ") + di.dli_sname);
    return p->by_handle.emplace(handle, k->second).first->second;
}

void queue_error(hsa_status_t status, hsa_queue_t*, void* data) {
    const char* m = nullptr;
    hsa_status_string(status, &m);
    std::fprintf(stderr, "tang_hip: AQL queue error: %s\n", m ? m : "unknown");
    ((std::atomic<int>*)data)->store(1);
}

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

// Device clock stamp (s_memrealtime, 100 MHz) of when this kernel ran.
__global__ void aql_stamp_kernel(unsigned long long* out) {
    if (threadIdx.x == 0)
        __hip_atomic_store(out, (unsigned long long)__builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// One HSA queue per device, plus the completion signal its sequences
// decrement.
struct AqlDev {
    Program* prog = nullptr;
    hsa_queue_t* queue = nullptr;
    hsa_signal_t done{};
    std::atomic<int> error{0};
    unsigned long long* stamps = nullptr;  // device: four clock stamps
    AqlSeq* stamp_seq[2] = {nullptr, nullptr};
    bool in_flight = false;
};

struct AqlPacket {
    uint64_t object;
    uint32_t grid[3];
    uint16_t block[3];
    uint32_t group_bytes, private_bytes;
    size_t karg_off;
};

struct AqlSeq {
    th_device* dev = nullptr;
    bool write_through = false;
    bool independent = false;  // no kernel reads what another kernel of the sequence writes
    std::vector<AqlPacket> packets;
    std::vector<char> kargs;     // host image of the kernarg segments
    char* kargs_dev = nullptr;   // device copy the packets point at
};

AqlSeq* aql_recording() { return g_recording; }

bool aql_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("TANG_HIP_DISPATCH");
        return !(e && (std::strcmp(e, "graph") == 0 || std::strcmp(e, "hip") == 0));
    }();
    return on;
}

static AqlDev* aql_dev(th_device* d) {
    if (d->aql) return d->aql;
    std::lock_guard<std::mutex> lock(g_mu);
    TH_HSA(hsa_init());  // reference-counted; HIP has initialised the runtime already
    AqlDev* a = new AqlDev;
    try {
        const hsa_agent_t agent = agent_of(d->ordinal);
        a->prog = program_for(agent);
        TH_HSA(hsa_queue_create(agent, QUEUE_PACKETS, HSA_QUEUE_TYPE_SINGLE, queue_error, &a->error, UINT32_MAX,
                                UINT32_MAX, &a->queue));
        TH_HSA(hsa_signal_create(0, 0, nullptr, &a->done));
        TH_HIP(hipMalloc((void**)&a->stamps, 4 * sizeof(unsigned long long)));
    } catch (...) {
        if (a->queue) (void)hsa_queue_destroy(a->queue);
        delete a;
        throw;
    }
    d->aql = a;
    return a;
}

void aql_record_launch(AqlSeq* seq, const void* kernel, dim3 grid, dim3 block, size_t shmem, const void* args,
                       size_t bytes) {
    AqlDev* a = aql_dev(seq->dev);
    const KernelInfo k = kernel_info(a->prog, kernel);
    if (seq->write_through && !k.write_through) {
        Dl_info di{};
        const char* name = dladdr(kernel, &di) && di.dli_sname ? di.dli_sname : "?";
        throw Error(TH_ERR_INVALID, std::string("kernel in a write-through sequence is not a write-through kernel: ") +
                                        name);
    }
    const size_t explicit_end = round_up(bytes, 8);
    size_t seg = std::max<size_t>(k.kernarg_bytes, bytes);
    const bool hidden = k.kernarg_bytes > explicit_end;
    TH_REQUIRE(!hidden || k.kernarg_bytes == explicit_end + HIDDEN_ARGS_BYTES,
               "kernel's kernarg segment does not match its parameters");
    TH_REQUIRE(block.x * block.y * block.z <= 1024 && block.x <= 0xFFFF, "bad block");
    const size_t off = round_up(seq->kargs.size(), KERNARG_ALIGN);
    seq->kargs.resize(off + round_up(seg, KERNARG_ALIGN), 0);
    char* dst = seq->kargs.data() + off;
    std::memcpy(dst, args, bytes);
    if (hidden) {  // block counts, group sizes and grid dimensions (code object v5 layout)
        char* h = dst + explicit_end;
        const uint32_t bc[3] = {grid.x, grid.y, grid.z};
        const uint16_t gs[3] = {(uint16_t)block.x, (uint16_t)block.y, (uint16_t)block.z};
        const uint16_t dims = grid.z > 1 || block.z > 1 ? 3 : (grid.y > 1 || block.y > 1 ? 2 : 1);
        std::memcpy(h, bc, sizeof bc);
        std::memcpy(h + 12, gs, sizeof gs);
        std::memcpy(h + 64, &dims, 2);
    }
    AqlPacket p;
    p.object = k.object;
    p.grid[0] = grid.x * block.x; p.grid[1] = grid.y * block.y; p.grid[2] = grid.z * block.z;
    p.block[0] = (uint16_t)block.x; p.block[1] = (uint16_t)block.y; p.block[2] = (uint16_t)block.z;
    p.group_bytes = k.group_bytes + (uint32_t)shmem;
    p.private_bytes = k.private_bytes;
    p.karg_off = off;
    TH_REQUIRE(p.group_bytes <= 160 * 1024, "workgroup memory exceeds the CU's LDS");
    seq->packets.push_back(p);
}

AqlSeq* aql_record(th_device* d, bool write_through, const std::function<void()>& enqueue, bool independent) {
    TH_REQUIRE(!g_recording, "nested AQL recording");
    aql_dev(d);
    AqlSeq* seq = new AqlSeq;
    seq->dev = d;
    seq->write_through = write_through;
    seq->independent = independent && write_through;
    // Anything other than a kernel launch would go to the stream: capture the
    // stream meanwhile and refuse a sequence that leaves nodes in the capture.
    hipGraph_t g = nullptr;
    try {
        TH_HIP(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal));
        g_recording = seq;
        try {
            enqueue();
        } catch (...) {
            g_recording = nullptr;
            hipGraph_t dummy;
            (void)hipStreamEndCapture(d->stream, &dummy);
            if (dummy) (void)hipGraphDestroy(dummy);
            throw;
        }
        g_recording = nullptr;
        TH_HIP(hipStreamEndCapture(d->stream, &g));
        size_t nodes = 0;
        TH_HIP(hipGraphGetNodes(g, nullptr, &nodes));
        (void)hipGraphDestroy(g);
        TH_REQUIRE(nodes == 0, "sequence enqueues stream operations other than kernel launches");
        TH_REQUIRE(!seq->packets.empty(), "empty sequence");
        TH_HIP(hipMalloc((void**)&seq->kargs_dev, seq->kargs.size()));
        TH_HIP(hipMemcpy(seq->kargs_dev, seq->kargs.data(), seq->kargs.size(), hipMemcpyHostToDevice));
    } catch (...) {
        aql_free(seq);
        throw;
    }
    return seq;
}

void aql_free(AqlSeq* seq) {
    if (!seq) return;
    try {
        if (seq->dev && seq->dev->aql) aql_wait(seq->dev);
    } catch (...) {
    }
    if (seq->kargs_dev) (void)hipFree(seq->kargs_dev);
    delete seq;
}

void aql_submit(const AqlSeq& seq, size_t repeat) {
    th_device* d = seq.dev;
    AqlDev* a = aql_dev(d);
    TH_REQUIRE(!a->error.load(), "AQL queue is in an error state");
    // earlier HIP work on the device stream comes first
    if (!a->in_flight) TH_HIP(hipStreamSynchronize(d->stream));
    hsa_queue_t* q = a->queue;
    const size_t np = seq.packets.size(), n = np * repeat;
    if (n == 0) return;
    // Inside a write-through sequence: no release (the values later kernels
    // read are already at the coherence point), but the agent-scope acquire
    // stays: it invalidates the XCD L2s, which may hold lines a kernel read
    // before an earlier kernel of the sequence rewrote them.  (Dropping it too
    // measured another 0.13-0.25 us per launch, but the memory model gives
    // no guarantee for plain loads then.)
    const uint16_t mid_rel = seq.write_through ? HSA_FENCE_SCOPE_NONE : HSA_FENCE_SCOPE_AGENT;
    // A sequence whose kernels read nothing another of its kernels writes
    // needs no acquire between them either.
    const uint16_t mid_acq = seq.independent ? HSA_FENCE_SCOPE_NONE : HSA_FENCE_SCOPE_AGENT;
    hsa_signal_add_relaxed(a->done, 1);
    a->in_flight = true;
    uint64_t idx = 0;
    const double t0 = now_s();
    for (size_t i = 0; i < n; i++) {
        const AqlPacket& p = seq.packets[i % np];
        // one producer (this thread): wait for a free slot, then take it, so a
        // failed wait leaves no reserved slot unwritten
        idx = hsa_queue_load_write_index_relaxed(q);
        while (idx - hsa_queue_load_read_index_scacquire(q) >= q->size) {
            if (a->error.load() || now_s() - t0 > WAIT_LIMIT_S) {
                a->error.store(1);  // its sequence is cut short: the queue is unusable from here
                throw Error(TH_ERR_HIP, "AQL queue does not drain");
            }
        }
        hsa_queue_store_write_index_relaxed(q, idx + 1);
        hsa_kernel_dispatch_packet_t* pk = (hsa_kernel_dispatch_packet_t*)q->base_address + (idx & (q->size - 1));
        const uint16_t setup = 3 << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS;
        pk->workgroup_size_x = p.block[0]; pk->workgroup_size_y = p.block[1]; pk->workgroup_size_z = p.block[2];
        pk->reserved0 = 0;
        pk->grid_size_x = p.grid[0]; pk->grid_size_y = p.grid[1]; pk->grid_size_z = p.grid[2];
        pk->private_segment_size = p.private_bytes;
        pk->group_segment_size = p.group_bytes;
        pk->kernel_object = p.object;
        pk->kernarg_address = seq.kargs_dev + p.karg_off;
        pk->reserved2 = 0;
        pk->completion_signal = i + 1 == n ? a->done : hsa_signal_t{0};
        const uint16_t acq = i == 0 ? HSA_FENCE_SCOPE_SYSTEM : mid_acq;
        const uint16_t rel = i + 1 == n ? HSA_FENCE_SCOPE_SYSTEM : mid_rel;
        const uint16_t header = (HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) |
                                (1 << HSA_PACKET_HEADER_BARRIER) | (acq << HSA_PACKET_HEADER_ACQUIRE_FENCE_SCOPE) |
                                (rel << HSA_PACKET_HEADER_RELEASE_FENCE_SCOPE);
        __atomic_store_n((uint32_t*)pk, (uint32_t)header | ((uint32_t)setup << 16), __ATOMIC_RELEASE);
        // doorbell every 256 packets, and at the ring's last slot, so that no
        // rung batch wraps around the end of the ring (queue interceptors,
        // such as a profiler's, copy a rung batch as one range)
        if ((i & 255) == 255 || ((idx + 1) & (q->size - 1)) == 0)
            hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)idx);
    }
    hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)idx);
}

void aql_wait(th_device* d) {
    AqlDev* a = d->aql;
    if (!a || !a->in_flight) return;
    const double t0 = now_s();
    while (hsa_signal_wait_scacquire(a->done, HSA_SIGNAL_CONDITION_EQ, 0, 1000000000ull, HSA_WAIT_STATE_ACTIVE) != 0) {
        if (a->error.load()) throw Error(TH_ERR_HIP, "AQL queue error");
        if (now_s() - t0 > WAIT_LIMIT_S) throw Error(TH_ERR_HIP, "AQL sequence did not complete");
    }
    a->in_flight = false;
}

void aql_stamp(th_device* d, int which) {
    AqlDev* a = aql_dev(d);
    if (!a->stamp_seq[which]) {
        unsigned long long* slot = a->stamps + which;
        a->stamp_seq[which] = aql_record(d, true, [&] {
            TH_LAUNCH(aql_stamp_kernel, dim3(1), dim3(64), 0, d->stream, slot);
        });
    }
    aql_submit(*a->stamp_seq[which]);
}

void aql_stamp_launch(th_device* d, int which) {
    TH_REQUIRE(which >= 0 && which < 4, "stamp slot out of range");
    AqlDev* a = aql_dev(d);
    TH_LAUNCH(aql_stamp_kernel, dim3(1), dim3(64), 0, d->stream, a->stamps + which);
}

float aql_stamped_ms(th_device* d) {
    aql_wait(d);
    unsigned long long t[2];
    TH_HIP(hipMemcpy(t, d->aql->stamps, sizeof t, hipMemcpyDeviceToHost));
    return (float)((double)(t[1] - t[0]) / 100e6 * 1e3);
}

float aql_stamp_span_ms(th_device* d) {
    aql_wait(d);
    unsigned long long t[2];
    TH_HIP(hipMemcpy(t, d->aql->stamps + 2, sizeof t, hipMemcpyDeviceToHost));
    return (float)((double)(t[1] - t[0]) / 100e6 * 1e3);
}

void aql_release(th_device* d) {
    AqlDev* a = d->aql;
    if (!a) return;
    try {
        aql_wait(d);
    } catch (...) {
    }
    for (AqlSeq*& s : a->stamp_seq) {
        if (s) {
            if (s->kargs_dev) (void)hipFree(s->kargs_dev);
            delete s;
        }
        s = nullptr;
    }
    if (a->stamps) (void)hipFree(a->stamps);
    (void)hsa_signal_destroy(a->done);
    (void)hsa_queue_destroy(a->queue);
    delete a;
    d->aql = nullptr;
    (void)hsa_shut_down();
}

}  // namespace th

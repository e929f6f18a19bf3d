// A C++ caller of the kvexp API (include/kvexp/attention.hpp, codec.hpp)
// linked against libkvexp_hip_cxx.so, calling it from an OpenMP parallel for
// the way the reference's bench calls attention_decode (src/bench.cpp:715-728:
// one call per job, n_threads = splits of that call, jobs spread over host
// threads). Built by compressed-kv-attention_amd/build.py with g++ -fopenmp;
// run by tests/test_gpu_cxx_api.py.
//
//   cxx_api_threads DIR [threads] [rounds]
//
// DIR/cases.txt lists one case per line:
//   name backend n_q dim seq n_threads split_tokens kx_bytes vx_bytes
// (backend 0 = Hip, 1 = HipDpbf16) with the files DIR/name.{q,k,v} (BF16),
// DIR/name.{kx,vx} (containers) and DIR/name.want (FP32 expected output).
// Every case runs with raw and with XKV inputs, `rounds` times, and every
// encode_bf16 / decode_bf16 of K runs as well; all results are compared bit
// for bit. Each host thread also checks the exception classes and messages
// of bad calls. Prints one summary line and exits non-zero on any mismatch.
#include "kvexp/attention.hpp"
#include "kvexp/codec.hpp"

#include <omp.h>

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

struct Case {
    std::string name;
    int backend = 0, n_q = 0, dim = 0, seq = 0, threads = 0, split = 0;
    std::vector<uint16_t> q, k, v;
    std::vector<uint8_t> kx, vx;
    std::vector<float> want;
};

template <class T> std::vector<T> load(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::vector<char> b((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    std::vector<T> out(b.size() / sizeof(T));
    if (!b.empty()) std::memcpy(out.data(), b.data(), out.size() * sizeof(T));
    return out;
}

std::mutex g_log_mu;
std::vector<std::string> g_log;
std::atomic<int> g_fail{0}, g_calls{0};

void failure(const std::string &msg) {
    g_fail.fetch_add(1);
    std::lock_guard<std::mutex> lock(g_log_mu);
    if (g_log.size() < 20) g_log.push_back(msg);
}

kvexp::Backend backend_of(int b) { return b == 0 ? kvexp::Backend::Hip : kvexp::Backend::HipDpbf16; }

// One job of the parallel for: case c with raw (xkv = false) or XKV inputs.
void run_attention(const Case &c, bool xkv) {
    std::vector<float> out(size_t(c.n_q) * size_t(c.dim), -1.0f);
    try {
        if (xkv)
            kvexp::attention_decode(backend_of(c.backend), c.q.data(), nullptr, nullptr, c.kx.data(), c.kx.size(),
                                    c.vx.data(), c.vx.size(), out.data(), c.n_q, c.dim, c.seq, c.threads, c.split);
        else
            kvexp::attention_decode(backend_of(c.backend), c.q.data(), c.k.data(), c.v.data(), nullptr, 0, nullptr, 0,
                                    out.data(), c.n_q, c.dim, c.seq, c.threads, c.split);
        g_calls.fetch_add(1);
    } catch (const std::exception &e) {
        failure(c.name + (xkv ? " xkv" : " raw") + ": threw " + e.what());
        return;
    }
    if (std::memcmp(out.data(), c.want.data(), out.size() * 4) != 0)
        failure(c.name + (xkv ? " xkv" : " raw") + ": output bits differ from the reference's");
}

void run_codec(const Case &c, int block) {
    try {
        const kvexp::EncodedTensor e = kvexp::encode_bf16(c.k.data(), c.seq, c.dim, block);
        g_calls.fetch_add(1);
        if (e.bytes != c.kx) failure(c.name + ": encode_bf16 bytes differ from the reference's");
        std::vector<uint16_t> back(c.k.size());
        kvexp::decode_bf16(e.bytes.data(), e.bytes.size(), c.seq, c.dim, back.data());
        g_calls.fetch_add(1);
        if (back != c.k) failure(c.name + ": decode_bf16(encode_bf16(k)) != k");
    } catch (const std::exception &e) {
        failure(c.name + ": codec threw " + e.what());
    }
}

// Runs fn and checks that it throws exactly an E whose message starts with `msg`.
template <class E, class F> void expect_throw(const char *what, const std::string &msg, F &&fn) {
    try {
        fn();
        failure(std::string(what) + ": did not throw");
    } catch (const E &e) {
        if (std::string(e.what()).rfind(msg, 0) != 0)
            failure(std::string(what) + ": message '" + e.what() + "', expected '" + msg + "'");
        else
            g_calls.fetch_add(1);
    } catch (const std::exception &e) {
        failure(std::string(what) + ": wrong exception class: " + e.what());
    }
}

// The reference's exception classes and texts for bad calls
// (dispatch.cpp:31-45, codec.cpp:40-52, scan.hpp:28-66,107-109).
void run_errors(const Case &c) {
    std::vector<float> out(size_t(c.n_q) * size_t(c.dim));
    using kvexp::Backend;
    expect_throw<std::invalid_argument>("null q", "attention_decode: bad argument", [&] {
        kvexp::attention_decode(Backend::Hip, nullptr, c.k.data(), c.v.data(), nullptr, 0, nullptr, 0, out.data(),
                                c.n_q, c.dim, c.seq, 1, c.split);
    });
    expect_throw<std::invalid_argument>("raw and xkv", "attention_decode: pass raw K and V or xkv K and V", [&] {
        kvexp::attention_decode(Backend::Hip, c.q.data(), c.k.data(), c.v.data(), c.kx.data(), c.kx.size(),
                                c.vx.data(), c.vx.size(), out.data(), c.n_q, c.dim, c.seq, 1, c.split);
    });
    expect_throw<std::runtime_error>("cpu backend", "CPU backend requested but not available", [&] {
        kvexp::attention_decode(Backend::Scalar, c.q.data(), c.k.data(), c.v.data(), nullptr, 0, nullptr, 0,
                                out.data(), c.n_q, c.dim, c.seq, 1, c.split);
    });
    expect_throw<std::runtime_error>("truncated container", "truncated xkv block header", [&] {
        kvexp::attention_decode(Backend::Hip, c.q.data(), nullptr, nullptr, c.kx.data(), 5, c.vx.data(),
                                c.vx.size(), out.data(), c.n_q, c.dim, c.seq, 1, c.split);
    });
    std::vector<uint8_t> bad = c.kx;
    bad[0] = 1; // mode byte 1 is no mode of the format
    expect_throw<std::runtime_error>("bad mode", "unknown xkv block mode", [&] {
        kvexp::attention_decode(Backend::Hip, c.q.data(), nullptr, nullptr, bad.data(), bad.size(), c.vx.data(),
                                c.vx.size(), out.data(), c.n_q, c.dim, c.seq, 1, c.split);
    });
    expect_throw<std::invalid_argument>("encode empty", "encode_bf16: empty input",
                                        [&] { (void)kvexp::encode_bf16(nullptr, c.seq, c.dim, c.split); });
    expect_throw<std::invalid_argument>("encode dim", "encode_bf16: head_dim must be a multiple of 4",
                                        [&] { (void)kvexp::encode_bf16(c.k.data(), 1, 6, c.split); });
}

} // namespace

int main(int argc, char **argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s DIR [threads] [rounds]\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const int nthreads = argc > 2 ? std::atoi(argv[2]) : 8;
    const int rounds = argc > 3 ? std::atoi(argv[3]) : 2;
    std::vector<Case> cases;
    {
        std::ifstream m(dir + "/cases.txt");
        std::string line;
        while (std::getline(m, line)) {
            if (line.empty()) continue;
            std::istringstream is(line);
            Case c;
            size_t kxb = 0, vxb = 0;
            is >> c.name >> c.backend >> c.n_q >> c.dim >> c.seq >> c.threads >> c.split >> kxb >> vxb;
            const std::string p = dir + "/" + c.name;
            c.q = load<uint16_t>(p + ".q");
            c.k = load<uint16_t>(p + ".k");
            c.v = load<uint16_t>(p + ".v");
            c.kx = load<uint8_t>(p + ".kx");
            c.vx = load<uint8_t>(p + ".vx");
            c.want = load<float>(p + ".want");
            if (c.kx.size() != kxb || c.vx.size() != vxb || c.want.size() != size_t(c.n_q) * c.dim)
                throw std::runtime_error("bad fixture " + c.name);
            cases.push_back(std::move(c));
        }
    }
    if (cases.empty()) {
        std::fprintf(stderr, "no cases in %s\n", dir.c_str());
        return 2;
    }
    // jobs: every case raw and XKV, `rounds` times; each case's codec once per round
    const int per_round = int(cases.size()) * 3;
    const int jobs = per_round * rounds;
    std::vector<int> ran(size_t(nthreads), 0);
    omp_set_dynamic(0);
    int got = 0;
#pragma omp parallel num_threads(nthreads)
    {
#pragma omp single
        got = omp_get_num_threads();
        const int tid = omp_get_thread_num();
        // every thread checks the error paths concurrently with the others' work
        run_errors(cases[size_t(tid) % cases.size()]);
#pragma omp for schedule(dynamic, 1)
        for (int j = 0; j < jobs; ++j) {
            const int r = j % per_round;
            const Case &c = cases[size_t(r / 3)];
            if (r % 3 == 2)
                run_codec(c, c.split);
            else
                run_attention(c, r % 3 == 1);
            ran[size_t(tid)]++;
        }
    }
    int active = 0;
    for (int n : ran) active += n > 0;
    std::printf("cxx_api_threads: %d threads (%d ran jobs), %zu cases, %d jobs, %d checked calls, %d failures\n", got,
                active, cases.size(), jobs, g_calls.load(), g_fail.load());
    for (const auto &s : g_log) std::printf("  FAIL %s\n", s.c_str());
    if (got != nthreads) return 3;
    return g_fail.load() == 0 ? 0 : 1;
}

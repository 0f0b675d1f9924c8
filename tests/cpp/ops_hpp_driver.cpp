// Compiled-C++ check of the drop-in layer include/ninfer_amd/ops.hpp: the reference's ninfer::ops call
// shapes (WorkspaceArena sized by gqa_attention_workspace_bytes(q_heads, tokens) as
// src/targets/qwen3_6/impl/runtime/layouts_impl.h:152 does, exceptions as the reference wrappers throw
// them) against the real library. TEST INFRASTRUCTURE: driven by tests/test_capi_cpu.py (mode
// `errors`, host validation only, no GPU) and tests/test_gpu_cpp_boundary.py (mode `run <dir>`: reads
// raw inputs written by the test, runs A1, argmax, greedy acceptance and the prefix commit on the GPU,
// writes the raw outputs back for comparison with the oracle).
#include "ninfer_amd/ops.hpp"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <functional>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

using namespace ninfer_amd;

namespace {

int failures = 0;

template <class E>
void expect_throw(const char* what, const std::function<void()>& f) {
    try {
        f();
    } catch (const E& e) {
        std::printf("ok %s: %s\n", what, e.what());
        return;
    } catch (const std::exception& e) {
        std::printf("FAIL %s: wrong exception type: %s\n", what, e.what());
        ++failures;
        return;
    }
    std::printf("FAIL %s: no exception\n", what);
    ++failures;
}

void* fake(uintptr_t p) { return reinterpret_cast<void*>(p); }

KVCacheLayerView fake_cache(uint32_t padded, uint32_t max_ctx) {
    KVCacheLayerView c;
    c.k = Tensor(fake(0x10000), DType::I8, {128, static_cast<int32_t>(padded), 8});
    c.v = Tensor(fake(0x10000), DType::I8, {128, static_cast<int32_t>(padded), 8});
    c.k_scale = Tensor(fake(0x10000), DType::FP16, {2, static_cast<int32_t>(padded), 8});
    c.v_scale = Tensor(fake(0x10000), DType::FP16, {2, static_cast<int32_t>(padded), 8});
    c.max_context = max_ctx;
    c.padded_context = padded;
    c.num_kv_heads = 8;
    c.head_dim = 128;
    c.dtype = DType::I8;
    c.quant_group = 64;
    return c;
}

int run_errors() {
    // reference call shapes of the workspace query
    const std::size_t verify = ops::gqa_attention_workspace_bytes(40, 4);
    const std::size_t mtp = ops::gqa_attention_workspace_bytes(24, 1);
    const std::size_t prompt = ops::gqa_attention_workspace_bytes(24, 2048);
    std::printf("workspace 40x4=%zu 24x1=%zu 24x2048=%zu\n", verify, mtp, prompt);
    if (verify == 0 || mtp == 0 || prompt != ops::gqa_attention_workspace_bytes(24, 32)) { ++failures; }
    expect_throw<std::invalid_argument>("workspace geometry", [] { (void)ops::gqa_attention_workspace_bytes(36, 4); });

    std::vector<unsigned char> arena_mem(verify + 4096);
    WorkspaceArena arena(reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(arena_mem.data()) + 255) & ~uintptr_t{255}),
                         verify);
    Tensor q(fake(0x10000), DType::BF16, {128, 40, 4}), k(fake(0x10000), DType::BF16, {128, 8, 4});
    Tensor pos(fake(0x10000), DType::I32, {4}), out(fake(0x10000), DType::BF16, {128, 40, 4});
    const float scale = 0.08838834764831845f;
    expect_throw<std::invalid_argument>("bad scale", [&] {
        ops::gqa_attention(q, k, k, pos, 0.0625f, fake_cache(4224, 4100), {1, 4100}, arena, out, nullptr);
    });
    expect_throw<std::invalid_argument>("bad envelope", [&] {
        ops::gqa_attention(q, k, k, pos, scale, fake_cache(4224, 4100), {0, 4100}, arena, out, nullptr);
    });
    expect_throw<std::overflow_error>("padded_context above int32", [&] {
        ops::gqa_attention(q, k, k, pos, scale, fake_cache(0x80000000u, 0x7FFFFFFFu), {1, 4100}, arena, out, nullptr);
    });
    Tensor q33(fake(0x10000), DType::BF16, {128, 40, 33, 2}), k33(fake(0x10000), DType::BF16, {128, 8, 33, 2});
    Tensor pos33(fake(0x10000), DType::I32, {33, 2}), out33(fake(0x10000), DType::BF16, {128, 40, 33, 2});
    expect_throw<std::runtime_error>("prompt route (T = 33) for two sequences", [&] {
        ops::gqa_attention(q33, k33, k33, pos33, scale, fake_cache(4224, 4100), {1, 4100}, arena, out33, nullptr);
    });
    expect_throw<std::invalid_argument>("arena too small for the envelope", [&] {
        WorkspaceArena tiny(arena_mem.data(), 256);
        ops::gqa_attention(q, k, k, pos, scale, fake_cache(4224, 4100), {1, 4100}, tiny, out, nullptr);
    });
    Tensor cnt(fake(0x10000), DType::I32, {1});
    expect_throw<std::invalid_argument>("commit envelope", [&] {
        ops::kv_cache_append_prefix(k, k, pos, cnt, {0, 5}, fake_cache(4224, 4100), nullptr);
    });
    CyclicKVCacheLayerView ring;
    ring.k = Tensor(fake(0x10000), DType::BF16, {128, 4096, 8});
    ring.v = ring.k;
    ring.capacity = 3000;
    ring.padded_capacity = 4096;
    ring.num_kv_heads = 8;
    ring.head_dim = 128;
    expect_throw<std::invalid_argument>("cyclic capacity", [&] {
        ops::kv_cache_append_prefix(k, k, pos, cnt, {0, 4}, ring, nullptr);
    });
    std::printf("%s\n", failures == 0 ? "ERRORS PASS" : "ERRORS FAIL");
    return failures == 0 ? 0 : 1;
}

// ---- GPU run -------------------------------------------------------------------------------------

std::vector<char> read_file(const std::string& path, std::size_t bytes) {
    std::ifstream f(path, std::ios::binary);
    std::vector<char> d(bytes);
    if (!f.read(d.data(), static_cast<std::streamsize>(bytes))) { throw std::runtime_error("short read: " + path); }
    return d;
}

void write_file(const std::string& path, const void* p, std::size_t bytes) {
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(p), static_cast<std::streamsize>(bytes));
}

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) { throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e)); }
}

struct Dev {
    void* p = nullptr;
    std::size_t n = 0;
    explicit Dev(std::size_t bytes) : n(bytes) { hip_ok(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc"); }
    Dev(const std::string& path, std::size_t bytes) : Dev(bytes) {
        const auto h = read_file(path, bytes);
        hip_ok(hipMemcpy(p, h.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy h2d");
    }
    ~Dev() { (void)hipFree(p); }
    void save(const std::string& path) const {
        std::vector<char> h(n);
        hip_ok(hipMemcpy(h.data(), p, n, hipMemcpyDeviceToHost), "hipMemcpy d2h");
        write_file(path, h.data(), n);
    }
};

int run_gpu(const std::string& dir) {
    // meta: L T max_context padded vocab K length commit_count
    std::ifstream meta(dir + "/meta.txt");
    int L, T, max_ctx, P, V, K, length, commit;
    if (!(meta >> L >> T >> max_ctx >> P >> V >> K >> length >> commit)) { throw std::runtime_error("bad meta"); }
    const int Hq = 40, Hkv = 8, D = 128;
    const std::size_t plane = static_cast<std::size_t>(D) * P * Hkv, splane = static_cast<std::size_t>(2) * P * Hkv;
    Dev q(dir + "/q.bin", static_cast<std::size_t>(D) * Hq * T * 2), k(dir + "/k.bin", static_cast<std::size_t>(D) * Hkv * T * 2),
        v(dir + "/v.bin", static_cast<std::size_t>(D) * Hkv * T * 2), pos(dir + "/positions.bin", T * 4u);
    Dev kc(dir + "/kc.bin", plane), vc(dir + "/vc.bin", plane), ks(dir + "/ks.bin", splane * 2), vs(dir + "/vs.bin", splane * 2);
    Dev out(static_cast<std::size_t>(D) * Hq * T * 2);
    KVCacheLayerView cache;
    cache.k = Tensor(kc.p, DType::I8, {D, P, Hkv});
    cache.v = Tensor(vc.p, DType::I8, {D, P, Hkv});
    cache.k_scale = Tensor(ks.p, DType::FP16, {2, P, Hkv});
    cache.v_scale = Tensor(vs.p, DType::FP16, {2, P, Hkv});
    cache.max_context = static_cast<uint32_t>(max_ctx);
    cache.padded_context = static_cast<uint32_t>(P);
    cache.num_kv_heads = Hkv;
    cache.head_dim = D;
    cache.dtype = DType::I8;
    cache.quant_group = 64;

    // the reference's arena sizing: the (q_heads, tokens) query plus the sampler's
    const std::size_t attn_bytes = ops::gqa_attention_workspace_bytes(Hq, T);
    const std::size_t samp_bytes = ops::sampling_workspace_bytes(V, K + 1);
    const std::size_t arena_bytes = attn_bytes + samp_bytes + 512;
    Dev arena_mem(arena_bytes);
    hip_ok(hipMemset(arena_mem.p, 0xFF, arena_bytes), "hipMemset arena");
    WorkspaceArena arena(arena_mem.p, arena_bytes);
    hipStream_t stream = nullptr;
    hip_ok(hipStreamCreate(&stream), "hipStreamCreate");

    Tensor tq(q.p, DType::BF16, {D, Hq, T}), tk(k.p, DType::BF16, {D, Hkv, T}), tv(v.p, DType::BF16, {D, Hkv, T});
    Tensor tpos(pos.p, DType::I32, {T}), tout(out.p, DType::BF16, {D, Hq, T});
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    ops::gqa_attention(tq, tk, tv, tpos, scale, cache, {1, static_cast<uint32_t>(max_ctx)}, arena, tout, stream);

    // acceptance: argmax over the verify columns, then greedy acceptance with a device config
    Dev logits(dir + "/logits.bin", static_cast<std::size_t>(V) * (K + 1) * 2), drafts(dir + "/drafts.bin", K * 4u);
    Dev target(static_cast<std::size_t>(K + 1) * 4), dlen(4), dtok(4), so(static_cast<std::size_t>(K + 1) * 4), ns(4),
        acc(4), stats(static_cast<std::size_t>(4 + K) * 8), cfg(sizeof(SamplingConfig));
    SamplingConfig host_cfg{};
    hip_ok(hipMemcpy(cfg.p, &host_cfg, sizeof host_cfg, hipMemcpyHostToDevice), "cfg");
    hip_ok(hipMemcpy(dlen.p, &length, 4, hipMemcpyHostToDevice), "length");
    hip_ok(hipMemset(stats.p, 0, stats.n), "stats");
    Tensor tlog(logits.p, DType::BF16, {V, K + 1}), ttarget(target.p, DType::I32, {K + 1});
    ops::argmax(tlog, ttarget, V, stream);
    Tensor tdr(drafts.p, DType::I32, {K}), tlen(dlen.p, DType::I32, {1}), ttok(dtok.p, DType::I32, {1}),
        tso(so.p, DType::I32, {K + 1}), tns(ns.p, DType::I32, {1}), tacc(acc.p, DType::I32, {1}),
        tst(stats.p, DType::I64, {4 + K});
    ops::speculative_accept_greedy_drafts(ttarget, tlog, tdr, tlen, ttok, tso, tns, tacc, tst, V,
                                          static_cast<const SamplingConfig*>(cfg.p), arena, stream);

    // commit the accepted prefix of a second set of K/V columns at the following rows
    Dev k2(dir + "/k2.bin", k.n), v2(dir + "/v2.bin", v.n), pos2(dir + "/positions2.bin", T * 4u), cnt(4);
    hip_ok(hipMemcpy(cnt.p, &commit, 4, hipMemcpyHostToDevice), "count");
    Tensor tk2(k2.p, DType::BF16, {D, Hkv, T}), tv2(v2.p, DType::BF16, {D, Hkv, T}), tpos2(pos2.p, DType::I32, {T}),
        tcnt(cnt.p, DType::I32, {1});
    ops::kv_cache_append_prefix(tk2, tv2, tpos2, tcnt, {0, static_cast<uint32_t>(T)}, cache, stream);
    hip_ok(hipStreamSynchronize(stream), "sync");
    hip_ok(hipStreamDestroy(stream), "stream destroy");

    out.save(dir + "/out.bin");
    kc.save(dir + "/kc_out.bin");
    vc.save(dir + "/vc_out.bin");
    ks.save(dir + "/ks_out.bin");
    vs.save(dir + "/vs_out.bin");
    target.save(dir + "/target_out.bin");
    so.save(dir + "/sampled_out.bin");
    dlen.save(dir + "/length_out.bin");
    dtok.save(dir + "/token_out.bin");
    stats.save(dir + "/stats_out.bin");
    std::printf("RUN PASS (attention workspace %zu bytes from the (q_heads, tokens) query)\n", attn_bytes);
    return 0;
}

} // namespace

int main(int argc, char** argv) {
    try {
        const std::string mode = argc > 1 ? argv[1] : "";
        if (mode == "errors") { return run_errors(); }
        if (mode == "run" && argc > 2) { return run_gpu(argv[2]); }
        std::fprintf(stderr, "usage: %s errors | run <dir>\n", argv[0]);
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: %s\n", e.what());
        return 1;
    }
}

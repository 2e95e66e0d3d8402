// A C++20 host program that drives libpadra_hip.so through include/padra_hip.h only, the
// way Padra's runtime drives the reference kernels: it fills the device control records
// (PrefillState as src/runtime/prefill_state.h:6-10 defines it, DecodeState as
// decode_control.cuh:3-6), builds the RoPE table with the host builder, allocates and
// clears the caches, launches, and reads the results back.
//
//   padra_caller <dir>
//
// Inputs (little-endian raw files written by tests/test_gpu_cpp_caller.py):
//   chain_meta.i32 {tokens, hidden, q_heads, kv_heads, capacity, base}
//   chain_x, chain_r, chain_gamma, chain_q, chain_k, chain_v, chain_qn, chain_kn (BF16 bits)
//   decode_meta.i32 {seqs, hidden, q_heads, kv_heads, capacity, vocab}
//   decode_embed, decode_r, decode_gamma, decode_q, decode_k, decode_v, decode_qn,
//   decode_kn (BF16 bits), decode_states.i32 [seqs][8]
// Part 1, the config-1 chunk: padra_ResidualNormQKRopeStore with positions from a device
// PrefillState (128-thread tree, BF16 cache of `capacity` rows), launched eagerly and then
// once more from a captured HIP graph after the chunk's state moves on the device.
// Part 2, the config-4 step: padra_EmbedResidualNormQKRopeStore with one DecodeState per
// sequence (256-thread tree, per-sequence BF16 caches `capacity` rows apart).
// Outputs: chain_out_* and decode_out_* (x, normalized, q, k, the cache rows the launch
// wrote, the flag), and replay_out_* for the graph replay.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <span>
#include <string>
#include <vector>

#include "padra_hip.h"

namespace {

std::string g_dir;

#define CHECK_HIP(e)                                                                       \
  do {                                                                                     \
    const hipError_t err_ = (e);                                                           \
    if (err_ != hipSuccess) {                                                              \
      std::fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(err_));    \
      std::exit(2);                                                                        \
    }                                                                                      \
  } while (0)
#define CHECK_PADRA(e)                                                                     \
  do {                                                                                     \
    const int st_ = (e);                                                                   \
    if (st_ != PADRA_OK) {                                                                 \
      std::fprintf(stderr, "%s:%d: padra status %d\n", __FILE__, __LINE__, st_);           \
      std::exit(3);                                                                        \
    }                                                                                      \
  } while (0)

template <class T> std::vector<T> read_file(const std::string &name) {
  std::ifstream f(g_dir + "/" + name, std::ios::binary | std::ios::ate);
  if (!f) {
    std::fprintf(stderr, "missing input %s\n", name.c_str());
    std::exit(4);
  }
  const auto bytes = static_cast<size_t>(f.tellg());
  std::vector<T> v(bytes / sizeof(T));
  f.seekg(0);
  f.read(reinterpret_cast<char *>(v.data()), static_cast<std::streamsize>(bytes));
  return v;
}

template <class T> void write_file(const std::string &name, std::span<const T> v) {
  std::ofstream f(g_dir + "/" + name, std::ios::binary);
  f.write(reinterpret_cast<const char *>(v.data()), static_cast<std::streamsize>(v.size_bytes()));
}

// A device buffer that frees itself.
template <class T> struct Device {
  T *p = nullptr;
  size_t n = 0;
  explicit Device(size_t count) : n(count) { CHECK_HIP(hipMalloc(&p, count * sizeof(T))); }
  explicit Device(const std::vector<T> &host) : Device(host.size()) {
    CHECK_HIP(hipMemcpy(p, host.data(), n * sizeof(T), hipMemcpyHostToDevice));
  }
  Device(const Device &) = delete;
  Device &operator=(const Device &) = delete;
  ~Device() { (void)hipFree(p); }
  std::vector<T> host() const {
    std::vector<T> v(n);
    CHECK_HIP(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
    return v;
  }
};

template <class T>
void dump(const std::string &name, const std::vector<T> &v) {
  write_file<T>(name, std::span<const T>(v));
}

// The cache rows [first, first + count) of a [rows][features] BF16 cache.
std::vector<uint16_t> rows_of(const Device<uint16_t> &cache, size_t features, size_t first,
                              size_t count) {
  std::vector<uint16_t> v(features * count);
  CHECK_HIP(hipMemcpy(v.data(), cache.p + first * features, v.size() * 2, hipMemcpyDeviceToHost));
  return v;
}

void chain_part(hipStream_t stream) {
  const auto meta = read_file<int32_t>("chain_meta.i32");
  const int tokens = meta[0], hidden = meta[1], hq = meta[2], hkv = meta[3], cap = meta[4],
            base = meta[5];
  const size_t features = static_cast<size_t>(hkv) * 128;
  std::vector<uint16_t> table(static_cast<size_t>(cap) * 128);
  CHECK_PADRA(padra_RopeTable(table.data(), cap, 128, 1e6f, 0, 16.f, 8192));
  Device<uint16_t> x(read_file<uint16_t>("chain_x")), r(read_file<uint16_t>("chain_r")),
      gamma(read_file<uint16_t>("chain_gamma")), q(read_file<uint16_t>("chain_q")),
      k(read_file<uint16_t>("chain_k")), v(read_file<uint16_t>("chain_v")),
      qn(read_file<uint16_t>("chain_qn")), kn(read_file<uint16_t>("chain_kn")), tab(table);
  Device<uint16_t> y(x.n), kc(static_cast<size_t>(cap) * features), vc(kc.n);
  CHECK_HIP(hipMemset(kc.p, 0, kc.n * 2));
  CHECK_HIP(hipMemset(vc.p, 0, vc.n * 2));
  Device<int> bad(1);
  CHECK_HIP(hipMemset(bad.p, 0, sizeof(int)));
  // The chunk's control record, as the runtime publishes it before the prefill graph runs.
  padra_PrefillState state{};
  state.base = base;
  state.prompt_offset = base;
  state.tokens = tokens;
  state.capacity = cap;
  state.committed = base;
  state.binding_epoch = 1;
  state.request_epoch = 1;
  state.valid = 1;
  Device<padra_PrefillState> dstate(std::vector<padra_PrefillState>{state});
  padra_Positions pos{};
  pos.mode = PADRA_POS_PREFILL;
  pos.prefill = dstate.p;
  pos.maximum = cap;
  pos.vocab = 98304;
  pos.binding_epoch = 1;
  padra_KVCache kv{};
  kv.format = PADRA_KV_BF16;
  kv.k = kc.p;
  kv.v = vc.p;
  kv.cap = cap;
  auto launch = [&] {
    CHECK_PADRA(padra_ResidualNormQKRopeStore(
        stream, x.p, r.p, y.p, gamma.p, hidden, PADRA_TREE_128, nullptr, q.p, k.p, v.p, qn.p,
        kn.p, tab.p, cap, &pos, tokens, hq, hkv, 128, 1e-6f, &kv, bad.p, PADRA_ACT_BF16));
  };
  launch();
  CHECK_HIP(hipStreamSynchronize(stream));
  dump("chain_out_x", x.host());
  dump("chain_out_y", y.host());
  dump("chain_out_q", q.host());
  dump("chain_out_k", k.host());
  dump("chain_out_kc", rows_of(kc, features, static_cast<size_t>(base), static_cast<size_t>(tokens)));
  dump("chain_out_vc", rows_of(vc, features, static_cast<size_t>(base), static_cast<size_t>(tokens)));
  dump("chain_out_bad", bad.host());

  // The same launch captured into a graph, replayed once the state has moved to the next
  // chunk position (base + tokens) on the device, from fresh inputs.
  hipGraph_t graph;
  hipGraphExec_t exec;
  CHECK_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
  launch();
  CHECK_HIP(hipStreamEndCapture(stream, &graph));
  CHECK_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
  state.base = base + tokens;
  state.prompt_offset = base + tokens;
  state.committed = base + tokens;
  CHECK_HIP(hipMemcpy(dstate.p, &state, sizeof state, hipMemcpyHostToDevice));
  for (auto [dst, name] : {std::pair{&x, "chain_x"}, {&q, "chain_q"}, {&k, "chain_k"}}) {
    const auto h = read_file<uint16_t>(name);
    CHECK_HIP(hipMemcpy(dst->p, h.data(), h.size() * 2, hipMemcpyHostToDevice));
  }
  CHECK_HIP(hipGraphLaunch(exec, stream));
  CHECK_HIP(hipStreamSynchronize(stream));
  dump("replay_out_x", x.host());
  dump("replay_out_y", y.host());
  dump("replay_out_q", q.host());
  dump("replay_out_k", k.host());
  dump("replay_out_kc", rows_of(kc, features, static_cast<size_t>(base + tokens),
                                static_cast<size_t>(tokens)));
  dump("replay_out_vc", rows_of(vc, features, static_cast<size_t>(base + tokens),
                                static_cast<size_t>(tokens)));
  dump("replay_out_bad", bad.host());
  CHECK_HIP(hipGraphExecDestroy(exec));
  CHECK_HIP(hipGraphDestroy(graph));
}

void decode_part(hipStream_t stream) {
  const auto meta = read_file<int32_t>("decode_meta.i32");
  const int seqs = meta[0], hidden = meta[1], hq = meta[2], hkv = meta[3], cap = meta[4],
            vocab = meta[5];
  const size_t features = static_cast<size_t>(hkv) * 128;
  std::vector<uint16_t> table(static_cast<size_t>(cap) * 128);
  CHECK_PADRA(padra_RopeTable(table.data(), cap, 128, 1e6f, 0, 16.f, 8192));
  const auto states = read_file<padra_DecodeState>("decode_states.i32");
  Device<uint16_t> embed(read_file<uint16_t>("decode_embed")), r(read_file<uint16_t>("decode_r")),
      gamma(read_file<uint16_t>("decode_gamma")), q(read_file<uint16_t>("decode_q")),
      k(read_file<uint16_t>("decode_k")), v(read_file<uint16_t>("decode_v")),
      qn(read_file<uint16_t>("decode_qn")), kn(read_file<uint16_t>("decode_kn")), tab(table);
  Device<padra_DecodeState> dstates(states);
  Device<uint16_t> x(static_cast<size_t>(seqs) * hidden), y(x.n),
      kc(static_cast<size_t>(seqs) * cap * features), vc(kc.n);
  CHECK_HIP(hipMemset(x.p, 0, x.n * 2));
  CHECK_HIP(hipMemset(kc.p, 0, kc.n * 2));
  CHECK_HIP(hipMemset(vc.p, 0, vc.n * 2));
  Device<int> bad(1);
  CHECK_HIP(hipMemset(bad.p, 0, sizeof(int)));
  padra_Positions pos{};
  pos.mode = PADRA_POS_DECODE;
  pos.decode = dstates.p;
  pos.maximum = cap;
  pos.vocab = vocab;
  pos.binding_epoch = 1;
  padra_KVCache kv{};
  kv.format = PADRA_KV_BF16;
  kv.k = kc.p;
  kv.v = vc.p;
  kv.cap = cap;
  kv.seq_stride = cap;
  CHECK_PADRA(padra_EmbedResidualNormQKRopeStore(
      stream, embed.p, vocab, nullptr, x.p, r.p, y.p, gamma.p, hidden, PADRA_TREE_256, nullptr,
      q.p, k.p, v.p, qn.p, kn.p, tab.p, cap, &pos, seqs, hq, hkv, 128, 1e-6f, &kv, bad.p));
  CHECK_HIP(hipStreamSynchronize(stream));
  dump("decode_out_x", x.host());
  dump("decode_out_y", y.host());
  dump("decode_out_q", q.host());
  dump("decode_out_k", k.host());
  // each sequence's one written row: sequence s, slot position % cap
  std::vector<uint16_t> krow, vrow;
  for (int s = 0; s < seqs; ++s) {
    const size_t row = static_cast<size_t>(s) * cap + static_cast<size_t>(states[s].position % cap);
    const auto kr = rows_of(kc, features, row, 1), vr = rows_of(vc, features, row, 1);
    krow.insert(krow.end(), kr.begin(), kr.end());
    vrow.insert(vrow.end(), vr.begin(), vr.end());
  }
  dump("decode_out_kc", krow);
  dump("decode_out_vc", vrow);
  dump("decode_out_bad", bad.host());
}

} // namespace

int main(int argc, char **argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s <dir>\n", argv[0]);
    return 1;
  }
  g_dir = argv[1];
  std::printf("%s\n", padra_version());
  hipStream_t stream;
  CHECK_HIP(hipStreamCreate(&stream));
  chain_part(stream);
  decode_part(stream);
  CHECK_HIP(hipStreamDestroy(stream));
  std::printf("ok\n");
  return 0;
}

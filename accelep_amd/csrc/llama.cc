// The Llama loop of AccelEP (src/llama_model.cc:209-247 Forward, :101-131 Generate,
// :325-380 create, :399-422 weights) on one MI355X.
//
// The call sequence per layer is the reference's: RMSNorm, q/k/v projections, RoPE on q and
// k, KV append, causal attention, o projection + residual, RMSNorm, gate/up, SiLU*up, down
// projection + residual; then the final RMSNorm of the last row and the LM head. What
// differs is where things live and how many passes there are (a decode step takes 5
// kernels per layer where the reference makes 15 device calls):
//  * q/k/v and gate/up are one matmul each over concatenated weights, storing into the
//    separate outputs (a column-split store); RoPE of q and k and both KV appends are one
//    kernel, and for a decode row (head_dim 64) that kernel is also the attention;
//  * for a one-row (decode) forward the RMSNorms and SiLU*up run inside the next int8 GEMV
//    (GemvPrologue), with the same bits as the separate passes a prompt uses;
//  * the residual adds run in the o and down projections' stores (c = acc + hidden, in
//    place), which gives the bits of the reference's MatMul + ResidualAdd pair;
//  * linear layers are int8 [in, out] with a per-output-column scale (the int8 GEMV for a
//    decode step, the int8-panel MFMA GEMM for a prompt) or fp32 [in, out];
//  * the sampler's xorshift state and the chosen ids stay in device memory, so a generate
//    call copies the ids back once and, with no eos id, never waits on the GPU in between;
//  * the decode step reads its position and id index from device memory and is replayed
//    from a HIP graph, so a token costs its kernels' time and not ~450 host launches.
// The tokenizer calls (src/llama_model.cc:183-205, :449-560) encode and decode on the host
// with ByteBpe (tokenizer.cc) around the same Generate.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "accel_llama.h"
#include "common.h"
#include "tokenizer.h"

namespace {

using namespace accel_hip;

thread_local std::string g_llama_error;

// One device allocation through the library heap (counted live, zero-filled), freed on destruction.
class DevBuf {
 public:
  DevBuf() = default;
  explicit DevBuf(size_t bytes) {
    if (accel_hip_allocate(bytes, &b_) != ACCEL_HIP_OK) Fail(ACCEL_HIP_BAD_ALLOC, accel_hip_last_error());
  }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : b_(o.b_) { o.b_ = AccelHipBuffer{}; }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      Release();
      b_ = o.b_;
      o.b_ = AccelHipBuffer{};
    }
    return *this;
  }
  ~DevBuf() { Release(); }

  template <typename T>
  T* as() const {
    return static_cast<T*>(b_.data);
  }
  const AccelHipBuffer& buffer() const { return b_; }
  bool empty() const { return b_.data == nullptr; }

  // Counted host-to-device copy (the reference uploads through Device::CopyHostToDevice).
  void Upload(const void* src, size_t bytes) {
    if (bytes != 0 && accel_hip_copy_h2d(b_, src, bytes) != ACCEL_HIP_OK) Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
  }

 private:
  void Release() {
    if (b_.data != nullptr) accel_hip_free(b_);
    b_ = AccelHipBuffer{};
  }
  AccelHipBuffer b_{};
};

// A linear layer held as [in, out]: fp32, or int8 with one scale per output column. The
// q/k/v projections share one such matrix (columns [q | k | v]) and so do gate/up
// ([gate | up]): one matmul fills both or all three outputs through a column-split store.
// Each part arrives through its own weight call; `filled` marks the parts loaded.
struct Linear {
  DevBuf f;      // fp32 [in, out]
  DevBuf q;      // int8 [in, out]
  DevBuf scale;  // fp32 [out]
  int64_t in = 0, out = 0;
  bool int8 = false;
  uint32_t filled = 0, parts = 1;
  bool ready() const { return (!f.empty() || !q.empty()) && filled == (1u << parts) - 1; }
};

// Where the HF weight of `kind` goes inside its Linear.
struct Part {
  Linear* linear = nullptr;
  int index = 0, parts = 1;
  int64_t col0 = 0, width = 0, in = 0, total = 0;
};

struct LayerWeights {
  DevBuf attn_norm, post_norm;
  Linear qkv, o, gu, down;
};

struct Model {
  AccelLlamaConfig cfg{};
  int32_t head_dim = 0;
  int32_t filled = 0;
  std::mutex mu;
  // Embedding: fp32 [vocab, hidden], or int8 [vocab, hidden] with a per-row scale.
  DevBuf embed_f, embed_q, embed_scale;
  DevBuf final_norm;
  Linear lm_head;
  DevBuf rope_cos, rope_sin;
  DevBuf hidden, normed, query, key, value, mixed, gate, up, logits;
  // words (int32): [0] embedding range flag, [1] sampler state, [2] position and [3] produced
  // count of the decode loop (read by the kernels of a replayed decode step).
  DevBuf chosen, prompt_ids, words;
  // The decode step (forward of the last chosen id + advance of [2], [3]) as a HIP graph,
  // captured on the second decode step of a generate (the first one stages the weights) and
  // replayed for every step after it. Dropped when a weight changes or the product mode does.
  void* decode_graph = nullptr;
  bool decode_graph_exact = false;
  bool decode_graph_pick = false;  // decode_graph starts with the greedy pick (GreedyEmbedKernel)
  bool decode_warm = false;
  // Timing marks of the decode step (ACCEL_LLAMA_DECODE_MARKS=<layer>, read at each capture):
  // the captured step records the event slots of accel_hip_event_record around the embedding,
  // that layer's five kernels, all the layers, the LM head's norm and product and the advance
  // (kMark*), and Generate records the sampler's start and end; the values left by the last
  // step of a generate time its parts (bench.py --decode-marks). The marks are event nodes of
  // the graph, so a marked step runs a little longer than an unmarked one. -1: no marks.
  int32_t decode_marks = -1;
  int32_t graph_marks = -1;  // the marks decode_graph was captured with
  // Decode-row fusions (accel_llama_set_fused_inputs): bit 0, RMSNorm and SiLU*up inside the
  // next GEMV; bit 1, RoPE + KV append + attention + combine as one kernel; bit 2 (fast mode,
  // over bit 1), the attention in fixed splits whose partials the o-projection GEMV combines.
  int32_t fuse = 7;
  // Attention partials of a decode step ([heads][context / 64 chunks][2 + head_dim]): owned
  // here so a captured step never points into a workspace that later grows.
  DevBuf attn_work;
  DevBuf attn_arrivals;  // uint32 per head, zero between decode attention launches
  DevBuf greedy_work;    // the greedy pick's count (zero between launches) and keys
  DevBuf greedy_keys;    // uint64 per 8-column tile of the LM head: the largest greedy key
  // The last forward's LM head stored greedy_keys for its logits (fused head, ApplyHead).
  bool head_keys = false;
  ByteBpe bpe;           // accel_llama_tokenizer
  DevBuf text_out;       // a completion's UTF-8 text on its way back (grows to the longest)

  enum MarkSlot : int32_t {
    kMarkStart = 0, kMarkEmbedded = 1, kMarkLayer = 2, kMarkQkv = 3, kMarkAttention = 4, kMarkO = 5,
    kMarkGateUp = 6, kMarkDown = 7, kMarkLayers = 8, kMarkHeadNorm = 9, kMarkHead = 10, kMarkAdvance = 11,
    kMarkSampleStart = 12, kMarkSampleEnd = 13,
    kMarkNode0 = 14, kMarkNode1 = 15  // two marks back to back: the cost of one event node
  };
  static int32_t MarksFromEnv() {
    const char* v = std::getenv("ACCEL_LLAMA_DECODE_MARKS");
    return v != nullptr && v[0] != 0 ? std::atoi(v) : -1;
  }
  // Records slot `slot` while the decode step is being captured with marks (`layer` -1: any).
  void Mark(int32_t slot, int32_t layer = -1) {
    if (decode_marks < 0 || !Capturing() || (layer >= 0 && layer != decode_marks)) return;
    if (accel_hip_event_record(slot) != ACCEL_HIP_OK) Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
  }

  void DropDecodeGraph() {
    if (decode_graph != nullptr) accel_hip_graph_destroy(decode_graph);
    decode_graph = nullptr;
    decode_warm = false;
  }
  ~Model() { DropDecodeGraph(); }
  std::vector<LayerWeights> layers;
  std::vector<DevBuf> k_cache, v_cache;

  hipStream_t stream() const { return Ctx().stream; }

  // The reference's forward makes 7 MatMul calls per layer and one for the LM head, each
  // noted as a kernel matmul (src/llama_model.cc:209-247, src/sim_device.cc:195,601). The
  // fused kernels here do the same products in fewer launches; the counter keeps the
  // reference's logical count, once per forward (prompt, forward_ids or decode step, also
  // when the step is a graph replay).
  void NoteForward() const { NoteKernelMatmuls(7 * static_cast<int64_t>(cfg.layers) + 1); }

  // Whether a decode step's int8 weights (the layers and the LM head) fit in three quarters of
  // MI355X's 256 MB last-level cache (MALL). Then the one-row GEMVs load their weights with
  // plain loads, so the next token finds them cached (SmolLM2-135M: 106 MB of layers and
  // 28 MB of LM head; 0.558 -> 0.539 ms per token at context 640). The KV cache is not
  // counted: a step reads its rows up to the position only, and the attention's plain loads
  // share the cache either way. A larger model streams its weights (nontemporal loads), which
  // keeps other data cached and reads HBM faster.
  bool cached_loads = false;
  void SetLoadPolicy() {
    const size_t h = static_cast<size_t>(cfg.hidden), inter = static_cast<size_t>(cfg.intermediate);
    const size_t q = static_cast<size_t>(cfg.heads) * head_dim, kv = static_cast<size_t>(cfg.kv_heads) * head_dim;
    const size_t layer = h * (q + 2 * kv) + q * h + h * 2 * inter + inter * h;
    const size_t total = static_cast<size_t>(cfg.layers) * layer + static_cast<size_t>(cfg.vocab) * h;
    cached_loads = total <= (size_t(192) << 20);
  }

  bool Ready() const {
    if ((embed_f.empty() && embed_q.empty()) || final_norm.empty() || !lm_head.ready()) return false;
    for (const LayerWeights& l : layers)
      if (l.attn_norm.empty() || l.post_norm.empty() || !l.qkv.ready() || !l.o.ready() || !l.gu.ready() ||
          !l.down.ready())
        return false;
    return true;
  }

  // c[m, out] = a[m, in] @ W with the epilogue in the store (residual, column split).
  void Apply(const Linear& w, const float* a, float* c, int64_t m, const Epilogue& e) {
    Context& ctx = Ctx();
    if (!w.q.empty()) {
      Q8View v;
      v.q = w.q.as<int8_t>();
      v.scale = w.scale.as<float>();
      v.mode = kScalePerCol;
      v.cached = cached_loads;
      if (ctx.exact_products) {
        LaunchExactMatmul(a, nullptr, v, c, m, w.in, w.out, e, ctx.stream);
      } else if (m <= 16) {
        if (GemvWantsGroups(m, w.in, w.out, v)) v.grouped = StagedGroupTiles(v.q, w.in, w.out, ctx.stream);
        else if (m <= 4) v.tiled = StagedColumnTiles(v.q, w.in, w.out, ctx.stream);
        LaunchGemvQ8(a, v, c, m, w.in, w.out, e, ctx.stream);
      } else {
        if (GemmWantsSmall(m, w.in, w.out, v)) v.bf16x16 = StagedBf16x16(v.q, w.in, w.out, ctx.stream);
        LaunchGemmF32(a, nullptr, v, c, m, w.in, w.out, e, ctx.stream);
      }
    } else if (ctx.exact_products) {
      LaunchExactMatmul(a, w.f.as<float>(), Q8View{}, c, m, w.in, w.out, e, ctx.stream);
    } else {
      LaunchGemmF32(a, w.f.as<float>(), Q8View{}, c, m, w.in, w.out, e, ctx.stream);
    }
  }

  // One row through an int8 weight on the GEMV, with the input transform done inside it.
  static constexpr int64_t kFusedNormMaxOut = 8192;
  bool Fusable(const Linear& w, int64_t m) const {
    return (fuse & 1) != 0 && m == 1 && !w.q.empty() && !Ctx().exact_products && w.in <= kGemvPrologueMaxK;
  }
  // The o-projection may read the split attention's partials (fuse bit 2).
  bool SplitAttention(const Linear& o) const {
    return (fuse & 4) != 0 && !o.q.empty() && !Ctx().exact_products && o.in <= kGemvPrologueMaxK &&
           o.in == static_cast<int64_t>(cfg.heads) * head_dim &&
           static_cast<int64_t>(cfg.heads) * DecodeAttentionSplits(cfg.context - 1) <= kGemvAttnMaxPairs;
  }
  void ApplyPrologue(const Linear& w, const float* x, float* c, const Epilogue& e, const GemvPrologue& pro) {
    Context& ctx = Ctx();
    Q8View v;
    v.q = w.q.as<int8_t>();
    v.scale = w.scale.as<float>();
    v.mode = kScalePerCol;
    v.cached = cached_loads;
    v.tiled = StagedColumnTiles(v.q, w.in, w.out, ctx.stream);
    LaunchGemvQ8(x, v, c, 1, w.in, w.out, e, ctx.stream, &pro);
  }
  // c = RMSNorm(x; norm) @ W: one kernel for a decode row, else the norm pass into `normed`.
  // A wide product (the LM head: 6144 workgroups) takes the separate pass too, rather than
  // every workgroup reading and normalizing the row again.
  // silu_split0 (only where SiluFold holds): the product's first column split is stored as
  // SiLU(v) (GemvPrologue::silu_split0).
  void ApplyNormed(const Linear& w, const float* x, const DevBuf& norm, float* c, int64_t m, const Epilogue& e,
                   int32_t norm_mark = -1, bool silu_split0 = false) {
    if (Fusable(w, m) && w.out <= kFusedNormMaxOut) {
      GemvPrologue pro;
      pro.rms_weight = norm.as<float>();
      pro.rms_eps = cfg.eps;
      pro.rms_after = true;
      pro.silu_split0 = silu_split0;
      ApplyPrologue(w, x, c, e, pro);
      return;
    }
    Q8View sv;
    if (SmallFusable(w, m, sv)) {
      SmallPrologue pro;
      pro.rms_weight = norm.as<float>();
      pro.rms_eps = cfg.eps;
      pro.silu_split0 = silu_split0;
      if (LaunchGemmQ8Small(x, sv, c, m, w.in, w.out, e, stream(), &pro)) return;
    }
    if (silu_split0) Fail(ACCEL_HIP_RUNTIME_ERROR, "SiLU store planned for a product that cannot take it");
    LaunchRmsNormRows(x, norm.as<float>(), normed.as<float>(), m, cfg.hidden, cfg.eps, stream());
    if (norm_mark >= 0) Mark(norm_mark);
    Apply(w, normed.as<float>(), c, m, e);
  }
  // A prompt's product (m > 16) on the small int8 GEMM, which can take the row's RMSNorm, the
  // multiply by up and the SiLU store as it splits A (fuse bit 1, fast mode; the staged copy is
  // built here on first use).
  bool SmallFusable(const Linear& w, int64_t m, Q8View& v) const {
    if ((fuse & 1) == 0 || m <= 16 || w.q.empty() || Ctx().exact_products) return false;
    v.q = w.q.as<int8_t>();
    v.scale = w.scale.as<float>();
    v.mode = kScalePerCol;
    v.cached = cached_loads;
    if (!GemmWantsSmall(m, w.in, w.out, v)) return false;
    v.bf16x16 = StagedBf16x16(v.q, w.in, w.out, Ctx().stream);
    return v.bf16x16 != nullptr;
  }
  // c = (SiLU(gate) * up) @ W: one kernel for a decode row, else SiLU*up in place first. With
  // silu_done the gate already holds SiLU(gate) (SiluFold) and the GEMV multiplies by up.
  void ApplySiluUp(const Linear& w, float* g, const float* u, float* c, int64_t m, const Epilogue& e,
                   bool silu_done = false) {
    if (Fusable(w, m)) {
      GemvPrologue pro;
      if (silu_done) pro.mul_up = u;
      else pro.silu_up = u;
      ApplyPrologue(w, g, c, e, pro);
      return;
    }
    if (silu_done) {
      Q8View sv;
      SmallPrologue pro;
      pro.mul = u;
      if (!SmallFusable(w, m, sv) || !LaunchGemmQ8Small(g, sv, c, m, w.in, w.out, e, stream(), &pro))
        Fail(ACCEL_HIP_RUNTIME_ERROR, "SiLU store planned for a down projection that cannot multiply by up");
      return;
    }
    LaunchSiluMul(g, u, m * cfg.intermediate, stream());
    Apply(w, g, c, m, e);
  }
  // A decode row's SiLU(gate) * up in two halves: the gate/up GEMV stores SiLU(gate) for its
  // gate columns (one expf per gate value) and the down GEMV multiplies by up, the same
  // operations as SiluMulKernel's, instead of every down workgroup forming SiLU per lane.
  // A prompt (m > 16) folds the same way when both products run on the small GEMM.
  bool SiluFold(const LayerWeights& l, int64_t m) const {
    if (m > 16) {
      Q8View gv, dv;
      const auto aligned = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
      return SmallFusable(l.gu, m, gv) && SmallFusable(l.down, m, dv) && aligned(hidden.as<float>()) &&
             aligned(l.post_norm.as<float>()) && aligned(gate.as<float>()) && aligned(up.as<float>());
    }
    return Fusable(l.gu, m) && l.gu.out <= kFusedNormMaxOut && l.gu.in % 2 == 0 && Fusable(l.down, m) &&
           l.down.in % 2 == 0;
  }
  // logits = RMSNorm(x; final_norm) @ lm_head for one row. Where the m = 1 GEMV runs the
  // product (fast mode, int8 head) the same kernel also stores the greedy keys of the logits
  // and, given the decode loop's state, advances it (no sampler scan over the logits and no
  // advance kernel). A wide head with a short row (one wave per tile, GemvWaveTileApplies)
  // with the fused inputs on takes the norm after the product in that kernel too; otherwise the
  // norm is a pass of its own (in the one-workgroup-per-tile kernel every workgroup would
  // reduce the row's sum of squares across its waves again: 13.3 us against 2.1 + 7.9).
  // Returns whether it advanced `state`.
  bool ApplyHead(const float* x, int32_t* state) {
    const bool side = !lm_head.q.empty() && !Ctx().exact_products && lm_head.in <= kGemvPrologueMaxK &&
                      lm_head.in % 2 == 0 && (lm_head.out + 7) / 8 <= kGreedyKeysMax;
    head_keys = side;
    if (side && Fusable(lm_head, 1) && GemvWaveTileApplies(1, lm_head.in, lm_head.out)) {
      // One wave per tile holds the whole row: the norm goes after the product, in the same kernel.
      GemvPrologue pro;
      pro.rms_weight = final_norm.as<float>();
      pro.rms_eps = cfg.eps;
      pro.rms_after = true;
      pro.greedy_keys = greedy_keys.as<uint64_t>();
      pro.advance = state;
      ApplyPrologue(lm_head, x, logits.as<float>(), Epilogue{}, pro);
      return state != nullptr;
    }
    LaunchRmsNormRows(x, final_norm.as<float>(), normed.as<float>(), 1, cfg.hidden, cfg.eps, stream());
    Mark(kMarkHeadNorm);
    if (!side) {
      Apply(lm_head, normed.as<float>(), logits.as<float>(), 1, Epilogue{});
      return false;
    }
    GemvPrologue pro;
    pro.greedy_keys = greedy_keys.as<uint64_t>();
    pro.advance = state;
    ApplyPrologue(lm_head, normed.as<float>(), logits.as<float>(), Epilogue{}, pro);
    return state != nullptr;
  }

  // Forward over `seq` ids at ids[id_offset ..] (device int32) from position `filled`
  // (src/llama_model.cc:209-247). Leaves the last row's logits in `logits`.
  // With `state` (device int32 [position, produced], seq == 1) the position and the id index
  // are read on the device, so the launches do not depend on the step. With `pick` as well,
  // the step starts by picking the greedy id from the previous head's keys into
  // ids[state[1]] and embedding it (one kernel, GreedyEmbedKernel) instead of embedding an id
  // a sampler wrote there. Returns whether the LM head advanced `state` (else the caller
  // launches the advance).
  bool Forward(const int32_t* ids, int32_t seq, int64_t id_offset, bool check_ids, int32_t* state = nullptr,
               bool pick = false) {
    if (ids == nullptr || seq <= 0 || filled < 0 || seq > cfg.context || filled > cfg.context - seq)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "forward exceeds context");
    const hipStream_t s = stream();
    const int64_t H = cfg.hidden, hd = head_dim, inter = cfg.intermediate;
    const int64_t pos = filled;
    int32_t* flag = words.as<int32_t>();
    Mark(kMarkNode0);
    Mark(kMarkNode1);
    Mark(kMarkStart);
    if (check_ids) Check(hipMemsetAsync(flag, 0, sizeof(int32_t), s), "hipMemsetAsync");
    if (pick && state != nullptr && seq == 1)
      LaunchGreedyEmbed(greedy_keys.as<uint64_t>(), (cfg.vocab + 7) / 8, state + 1, embed_q.as<int8_t>(),
                        embed_scale.as<float>(), embed_f.as<float>(), logits.as<float>(), const_cast<int32_t*>(ids),
                        hidden.as<float>(), H, s);
    else
      LaunchEmbedding(state != nullptr ? ids : ids + id_offset, embed_f.as<float>(), embed_q.as<int8_t>(),
                      embed_scale.as<float>(), hidden.as<float>(), seq, H, cfg.vocab, flag, s,
                      state != nullptr ? state + 1 : nullptr);
    Mark(kMarkEmbedded);
    if (check_ids) {
      int32_t bad = 0;
      Check(hipMemcpyAsync(&bad, flag, sizeof(bad), hipMemcpyDeviceToHost, s), "hipMemcpyAsync");
      Check(hipStreamSynchronize(s), "hipStreamSynchronize");
      if (bad != 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "token id is outside the vocabulary");
    }
    const int64_t q_out = static_cast<int64_t>(cfg.heads) * hd, kv_out = static_cast<int64_t>(cfg.kv_heads) * hd;
    Epilogue qkv;  // [q | k | v] -> query, key, value
    qkv.split[0] = q_out;
    qkv.split[1] = q_out + kv_out;
    qkv.c2 = key.as<float>();
    qkv.c3 = value.as<float>();
    Epilogue gu;  // [gate | up] -> gate, up
    gu.split[0] = inter;
    gu.split[1] = 2 * inter;
    gu.c2 = up.as<float>();
    Epilogue residual;  // c = acc + hidden, written over hidden
    residual.residual = hidden.as<float>();
    for (int32_t li = 0; li < cfg.layers; ++li) {
      LayerWeights& l = layers[static_cast<size_t>(li)];
      float* kc = k_cache[static_cast<size_t>(li)].as<float>();
      float* vc = v_cache[static_cast<size_t>(li)].as<float>();
      Mark(kMarkLayer, li);
      ApplyNormed(l.qkv, hidden.as<float>(), l.attn_norm, query.as<float>(), seq, qkv);
      Mark(kMarkQkv, li);
      const int splits =
          seq == 1 && SplitAttention(l.o)
              ? LaunchDecodeSplitAttention(query.as<float>(), key.as<float>(), value.as<float>(), kc, vc,
                                           rope_cos.as<float>(), rope_sin.as<float>(), pos, cfg.heads, cfg.kv_heads,
                                           hd, s, state, cfg.context - 1, attn_work.as<float>(),
                                           attn_work.buffer().bytes)
              : 0;
      if (splits > 0) {
        Mark(kMarkAttention, li);
        GemvPrologue pro;
        pro.attn_partial = attn_work.as<float>();
        pro.attn_splits = splits;
        ApplyPrologue(l.o, attn_work.as<float>(), hidden.as<float>(), residual, pro);
        Mark(kMarkO, li);
        const bool silu_fold = SiluFold(l, seq);
        ApplyNormed(l.gu, hidden.as<float>(), l.post_norm, gate.as<float>(), seq, gu, -1, silu_fold);
        Mark(kMarkGateUp, li);
        ApplySiluUp(l.down, gate.as<float>(), up.as<float>(), hidden.as<float>(), seq, residual, silu_fold);
        Mark(kMarkDown, li);
        continue;
      }
      if (seq != 1 || (fuse & 2) == 0 || !LaunchDecodeAttention(query.as<float>(), key.as<float>(), value.as<float>(), kc, vc,
                                             rope_cos.as<float>(), rope_sin.as<float>(), mixed.as<float>(), pos,
                                             cfg.heads, cfg.kv_heads, hd, s, state, cfg.context - 1,
                                             attn_work.as<float>(), attn_work.buffer().bytes,
                                             attn_arrivals.as<uint32_t>())) {
        LaunchRopeAppend(query.as<float>(), key.as<float>(), value.as<float>(), kc, vc, rope_cos.as<float>(),
                         rope_sin.as<float>(), seq, cfg.heads, cfg.kv_heads, hd, pos, s, state);
        LaunchAttention(query.as<float>(), kc, vc, mixed.as<float>(), seq, pos, cfg.heads, cfg.kv_heads, hd, s,
                        state, cfg.context - 1, attn_work.as<float>(), attn_work.buffer().bytes,
                        !Ctx().exact_products);
      }
      Mark(kMarkAttention, li);
      Apply(l.o, mixed.as<float>(), hidden.as<float>(), seq, residual);
      Mark(kMarkO, li);
      const bool silu_fold = SiluFold(l, seq);
      ApplyNormed(l.gu, hidden.as<float>(), l.post_norm, gate.as<float>(), seq, gu, -1, silu_fold);
      Mark(kMarkGateUp, li);
      ApplySiluUp(l.down, gate.as<float>(), up.as<float>(), hidden.as<float>(), seq, residual, silu_fold);
      Mark(kMarkDown, li);
    }
    Mark(kMarkLayers);
    const bool advanced = ApplyHead(hidden.as<float>() + static_cast<int64_t>(seq - 1) * H, state);
    Mark(kMarkHead);
    return advanced;
  }

  // One decode step: forward of chosen[produced] at `position` (with `pick`, chosen[produced]
  // is first picked from the previous head's greedy keys), then both advance. The first call
  // runs it directly (staging the weights and sizing the workspaces), the second captures it
  // into a graph, and later calls replay the graph.
  void DecodeStep(int32_t* state, bool pick = false) {
    const bool exact = Ctx().exact_products;
    decode_marks = MarksFromEnv();
    if (decode_graph != nullptr && (decode_graph_exact != exact || graph_marks != decode_marks ||
                                    decode_graph_pick != pick || !GraphIsCurrent(decode_graph)))
      DropDecodeGraph();
    // ACCEL_LLAMA_EAGER=1 launches every step directly (a profiler then sees each dispatch).
    static const bool eager = [] {
      const char* v = std::getenv("ACCEL_LLAMA_EAGER");
      return v != nullptr && v[0] == '1';
    }();
    if (eager || (decode_graph == nullptr && !decode_warm)) {
      if (!Forward(chosen.as<int32_t>(), 1, 0, false, state, pick)) LaunchAdvance(state, stream());
      decode_warm = true;
      return;
    }
    if (decode_graph == nullptr) {
      if (accel_hip_capture_begin() != ACCEL_HIP_OK) Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
      try {
        if (!Forward(chosen.as<int32_t>(), 1, 0, false, state, pick)) {
          LaunchAdvance(state, stream());
          Mark(kMarkAdvance);
        }
      } catch (...) {
        void* broken = nullptr;
        accel_hip_capture_end(&broken);
        if (broken != nullptr) accel_hip_graph_destroy(broken);
        throw;
      }
      if (accel_hip_capture_end(&decode_graph) != ACCEL_HIP_OK) Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
      decode_graph_exact = exact;
      decode_graph_pick = pick;
      graph_marks = decode_marks;
    }
    if (accel_hip_graph_launch(decode_graph, 1) != ACCEL_HIP_OK) Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
  }

  // src/llama_model.cc:101-131. on_token (may be null) receives each id after it is sampled
  // and before the eos check.
  void Generate(const int32_t* prompt, int32_t prompt_count, int32_t max_new, int32_t eos_id, float temperature,
                uint32_t seed, int32_t top_k, int32_t* out_ids, int32_t* out_count, AccelLlamaTokenFn on_token,
                void* user) {
    filled = 0;
    if (prompt == nullptr || prompt_count <= 0 || prompt_count > cfg.context)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "forward exceeds context");
    prompt_ids.Upload(prompt, static_cast<size_t>(prompt_count) * sizeof(int32_t));
    Forward(prompt_ids.as<int32_t>(), prompt_count, 0, true);
    NoteForward();
    filled = prompt_count;
    const uint32_t rng0 = seed == 0 ? 0x6d2b79f5u : seed;
    uint32_t* rng = words.as<uint32_t>() + 1;
    Check(hipMemcpyAsync(rng, &rng0, sizeof(rng0), hipMemcpyHostToDevice, stream()), "hipMemcpyAsync");
    Check(hipStreamSynchronize(stream()), "hipStreamSynchronize");
    int32_t* state = words.as<int32_t>() + 2;
    const int32_t state0[2] = {filled, 0};
    Check(hipMemcpyAsync(state, state0, sizeof(state0), hipMemcpyHostToDevice, stream()), "hipMemcpyAsync");
    Check(hipStreamSynchronize(stream()), "hipStreamSynchronize");
    int32_t produced = 0;
    // Greedy with the head's keys and no id needed on the host between steps: each decode step
    // starts by picking its id from the previous head's keys (GreedyEmbedKernel), so no sampler
    // kernel runs between the steps. The picks and forwards run in the same order as with one.
    const bool pick = !(temperature > 0.f) && head_keys && eos_id < 0 && on_token == nullptr;
    for (int32_t step = 0; step < max_new; ++step) {
      if (produced >= cfg.context) Fail(ACCEL_HIP_INVALID_ARGUMENT, "generation exceeded the token buffer");
      const bool mark_sample = decode_marks >= 0 && decode_graph != nullptr;  // steps that replay the marked graph
      if (!pick) {
        if (mark_sample && accel_hip_event_record(kMarkSampleStart) != ACCEL_HIP_OK)
          Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
        if (!(temperature > 0.f) && head_keys)
          LaunchGreedyKeys(greedy_keys.as<uint64_t>(), (cfg.vocab + 7) / 8, logits.as<float>(), chosen.as<int32_t>(),
                           state + 1, stream());
        else
          LaunchSampleToken(logits.as<float>(), chosen.as<int32_t>(), cfg.vocab, temperature, rng, top_k, stream(),
                            state + 1, greedy_work.as<uint32_t>(), greedy_work.buffer().bytes);
        if (mark_sample && accel_hip_event_record(kMarkSampleEnd) != ACCEL_HIP_OK)
          Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
      } else if (filled >= cfg.context) {
        // The last id, with no forward after it.
        LaunchGreedyKeys(greedy_keys.as<uint64_t>(), (cfg.vocab + 7) / 8, logits.as<float>(), chosen.as<int32_t>(),
                         state + 1, stream());
      }
      produced += 1;
      if (eos_id >= 0 || on_token != nullptr) {
        // Only an eos id or a token callback needs the chosen id on the host before the next
        // step (an uncounted read, as the reference's host reads it through a raw pointer).
        int32_t id = -1;
        Check(hipMemcpyAsync(&id, chosen.as<int32_t>() + produced - 1, sizeof(id), hipMemcpyDeviceToHost, stream()),
              "hipMemcpyAsync");
        Check(hipStreamSynchronize(stream()), "hipStreamSynchronize");
        if (on_token != nullptr) on_token(id, user);
        if (id == eos_id) break;
      }
      if (filled >= cfg.context) break;
      DecodeStep(state, pick);
      NoteForward();
      filled += 1;
    }
    if (produced > 0 && accel_hip_copy_d2h(out_ids, chosen.buffer(), static_cast<size_t>(produced) * sizeof(int32_t)) !=
                            ACCEL_HIP_OK)
      Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
    *out_count = produced;
  }

  // src/llama_model.cc:133-148: the text goes to the host through device memory, so its copy
  // back is a counted one, like the ids'.
  void CopyOutText(const std::string& text, char* out_text, int32_t cap, int32_t* out_len) {
    if (out_text == nullptr || out_len == nullptr || cap < 0 || static_cast<int64_t>(text.size()) > cap)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "completion text buffer is too small");
    *out_len = static_cast<int32_t>(text.size());
    if (text.empty()) return;
    if (text_out.buffer().bytes < text.size()) text_out = DevBuf(text.size());
    Check(hipMemcpyAsync(text_out.as<char>(), text.data(), text.size(), hipMemcpyHostToDevice, stream()),
          "hipMemcpyAsync");
    if (accel_hip_copy_d2h(out_text, text_out.buffer(), text.size()) != ACCEL_HIP_OK)
      Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
  }

  // src/llama_model.cc:183-206: encode the prompt, generate, decode the ids without special
  // tokens.
  void Complete(const char* prompt, int32_t prompt_len, int32_t max_new, int32_t eos_id, float temperature,
                uint32_t seed, int32_t top_k, char* out_text, int32_t out_text_cap, int32_t* out_text_len,
                int32_t* out_ids, int32_t out_ids_cap, int32_t* out_count, int32_t* prompt_tokens,
                AccelLlamaTokenFn on_token, void* user) {
    if (!bpe.loaded()) Fail(ACCEL_HIP_INVALID_ARGUMENT, "tokenizer is not loaded");
    if (prompt_len < 0 || (prompt_len > 0 && prompt == nullptr) || out_ids == nullptr || out_count == nullptr ||
        prompt_tokens == nullptr || out_ids_cap < max_new)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "invalid complete");
    const std::vector<int32_t> ids =
        bpe.Encode(prompt_len == 0 ? std::string_view() : std::string_view(prompt, static_cast<size_t>(prompt_len)));
    if (ids.empty()) Fail(ACCEL_HIP_INVALID_ARGUMENT, "prompt encoded to no tokens");
    if (static_cast<int32_t>(ids.size()) > cfg.context) Fail(ACCEL_HIP_INVALID_ARGUMENT, "prompt exceeds context");
    Generate(ids.data(), static_cast<int32_t>(ids.size()), max_new, eos_id, temperature, seed, top_k, out_ids,
             out_count, on_token, user);
    // out_ids holds what the device chose (copied back by Generate).
    const std::string text = bpe.Decode(out_ids, *out_count, true);
    CopyOutText(text, out_text, out_text_cap, out_text_len);
    *prompt_tokens = static_cast<int32_t>(ids.size());
  }
};

bool IsNorm(int32_t kind) {
  return kind == ACCEL_W_FINAL_NORM || kind == ACCEL_W_ATTN_NORM || kind == ACCEL_W_POST_NORM;
}

// Expected HF shape of a weight kind (src/llama_model.cc:290-318).
bool ShapeOk(const Model& m, int32_t kind, int64_t rows, int64_t cols) {
  const int64_t H = m.cfg.hidden, qo = static_cast<int64_t>(m.cfg.heads) * m.head_dim,
                ko = static_cast<int64_t>(m.cfg.kv_heads) * m.head_dim, I = m.cfg.intermediate;
  switch (kind) {
    case ACCEL_W_EMBED:
    case ACCEL_W_LM_HEAD:
      return rows == m.cfg.vocab && cols == H;
    case ACCEL_W_FINAL_NORM:
    case ACCEL_W_ATTN_NORM:
    case ACCEL_W_POST_NORM:
      return rows == H && cols == 1;
    case ACCEL_W_Q:
      return rows == qo && cols == H;
    case ACCEL_W_K:
    case ACCEL_W_V:
      return rows == ko && cols == H;
    case ACCEL_W_O:
      return rows == H && cols == qo;
    case ACCEL_W_DOWN:
      return rows == H && cols == I;
    case ACCEL_W_GATE:
    case ACCEL_W_UP:
      return rows == I && cols == H;
    default:
      return false;
  }
}

Part PartOf(Model& m, int32_t kind, int32_t layer) {
  const int64_t H = m.cfg.hidden, qo = static_cast<int64_t>(m.cfg.heads) * m.head_dim,
                ko = static_cast<int64_t>(m.cfg.kv_heads) * m.head_dim, I = m.cfg.intermediate;
  Part p;
  if (kind == ACCEL_W_LM_HEAD) {
    p.linear = &m.lm_head;
    p.width = p.total = m.cfg.vocab;
    p.in = H;
    return p;
  }
  if (layer < 0 || layer >= m.cfg.layers) return p;
  LayerWeights& l = m.layers[static_cast<size_t>(layer)];
  switch (kind) {
    case ACCEL_W_Q:
    case ACCEL_W_K:
    case ACCEL_W_V:
      p.linear = &l.qkv;
      p.parts = 3;
      p.index = kind - ACCEL_W_Q;
      p.col0 = kind == ACCEL_W_Q ? 0 : kind == ACCEL_W_K ? qo : qo + ko;
      p.width = kind == ACCEL_W_Q ? qo : ko;
      p.in = H;
      p.total = qo + 2 * ko;
      break;
    case ACCEL_W_O:
      p.linear = &l.o;
      p.width = p.total = H;
      p.in = qo;
      break;
    case ACCEL_W_GATE:
    case ACCEL_W_UP:
      p.linear = &l.gu;
      p.parts = 2;
      p.index = kind - ACCEL_W_GATE;
      p.col0 = kind == ACCEL_W_GATE ? 0 : I;
      p.width = I;
      p.in = H;
      p.total = 2 * I;
      break;
    case ACCEL_W_DOWN:
      p.linear = &l.down;
      p.width = p.total = H;
      p.in = I;
      break;
    default:
      break;
  }
  return p;
}

// Writes one part (its [in, width] block, already transposed) into its Linear.
void UploadPart(const Part& p, bool int8, const void* block, const float* scale) {
  Linear& w = *p.linear;
  if (w.f.empty() && w.q.empty()) {
    w.in = p.in;
    w.out = p.total;
    w.int8 = int8;
    w.parts = static_cast<uint32_t>(p.parts);
    w.filled = 0;
    if (int8) {
      w.q = DevBuf(static_cast<size_t>(p.in * p.total));
      w.scale = DevBuf(static_cast<size_t>(p.total) * sizeof(float));
    } else {
      w.f = DevBuf(static_cast<size_t>(p.in * p.total) * sizeof(float));
    }
  } else if (w.int8 != int8) {
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "a projection group mixes int8 and float weights");
  }
  const size_t elem = int8 ? 1 : sizeof(float);
  char* base = int8 ? w.q.as<char>() : w.f.as<char>();
  // On the library stream, behind the allocation's zero-fill (a stream-ordered memset there):
  // a copy on another stream could land first and be zeroed over.
  const hipStream_t s = Ctx().stream;
  NoteDeviceWrite(base, static_cast<size_t>(p.in * p.total) * elem);  // drops a staged copy of the old bytes
  Check(hipMemcpy2DAsync(base + p.col0 * elem, static_cast<size_t>(p.total) * elem, block,
                         static_cast<size_t>(p.width) * elem, static_cast<size_t>(p.width) * elem,
                         static_cast<size_t>(p.in), hipMemcpyHostToDevice, s),
        "hipMemcpy2DAsync");
  if (int8)
    Check(hipMemcpyAsync(w.scale.as<float>() + p.col0, scale, static_cast<size_t>(p.width) * sizeof(float),
                         hipMemcpyHostToDevice, s),
          "hipMemcpyAsync");
  // The host blocks may be temporaries of the caller: wait until they have been read.
  Check(hipStreamSynchronize(s), "hipStreamSynchronize");
  NoteBytesToDevice(static_cast<size_t>(p.in * p.width) * elem);
  if (int8) NoteBytesToDevice(static_cast<size_t>(p.width) * sizeof(float));
  w.filled |= 1u << p.index;
  // A complete int8 projection gets its decode GEMV tiles now, at load, not in the first step.
  if (int8 && w.ready() && StagedColumnTiles(w.q.as<int8_t>(), w.in, w.out, s) == nullptr)
    Fail(ACCEL_HIP_RUNTIME_ERROR, "staging a projection's GEMV tiles failed");
}

DevBuf* NormSlot(Model& m, int32_t kind, int32_t layer) {
  if (kind == ACCEL_W_FINAL_NORM) return &m.final_norm;
  if (layer < 0 || layer >= m.cfg.layers) return nullptr;
  if (kind == ACCEL_W_ATTN_NORM) return &m.layers[static_cast<size_t>(layer)].attn_norm;
  if (kind == ACCEL_W_POST_NORM) return &m.layers[static_cast<size_t>(layer)].post_norm;
  return nullptr;
}

// [rows, cols] -> [cols, rows] on the host.
template <typename T>
std::vector<T> Transposed(const T* src, int64_t rows, int64_t cols) {
  std::vector<T> dst(static_cast<size_t>(rows * cols));
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) dst[static_cast<size_t>(c * rows + r)] = src[r * cols + c];
  return dst;
}

template <typename F>
int Run(F f) {
  try {
    f();
    g_llama_error.clear();
    return 0;
  } catch (const Error& e) {
    g_llama_error = e.message;
  } catch (const std::bad_alloc&) {
    g_llama_error = "out of memory";
  } catch (const std::exception& e) {
    g_llama_error = e.what();
  }
  return 1;
}

Model* Get(AccelLlama* handle) { return reinterpret_cast<Model*>(handle); }

}  // namespace

extern "C" {

ACCEL_LLAMA_API AccelLlama* accel_llama_create(const AccelLlamaConfig* config) {
  if (config == nullptr || config->vocab <= 0 || config->hidden <= 0 || config->layers <= 0 || config->heads <= 0 ||
      config->kv_heads <= 0 || config->intermediate <= 0 || config->context <= 0 ||
      config->hidden % config->heads != 0 || config->heads % config->kv_heads != 0) {
    g_llama_error = "invalid llama config";
    return nullptr;
  }
  Model* made = nullptr;
  const int rc = Run([&] {
    auto m = std::make_unique<Model>();
    m->cfg = *config;
    m->head_dim = config->hidden / config->heads;
    m->layers.resize(static_cast<size_t>(config->layers));
    m->SetLoadPolicy();
    // RoPE tables in double, as src/llama_model.cc:333-349 builds them.
    const int32_t dim = m->head_dim, half = dim / 2;
    const size_t ctx = static_cast<size_t>(config->context);
    std::vector<float> cs(ctx * static_cast<size_t>(dim)), sn(ctx * static_cast<size_t>(dim));
    for (int32_t pos = 0; pos < config->context; ++pos)
      for (int32_t i = 0; i < half; ++i) {
        const double inv = 1.0 / std::pow(static_cast<double>(config->rope_theta), (2.0 * i) / static_cast<double>(dim));
        const double angle = static_cast<double>(pos) * inv;
        const size_t at = static_cast<size_t>(pos) * static_cast<size_t>(dim) + static_cast<size_t>(i);
        cs[at] = cs[at + static_cast<size_t>(half)] = static_cast<float>(std::cos(angle));
        sn[at] = sn[at + static_cast<size_t>(half)] = static_cast<float>(std::sin(angle));
      }
    m->rope_cos = DevBuf(cs.size() * sizeof(float));
    m->rope_cos.Upload(cs.data(), cs.size() * sizeof(float));
    m->rope_sin = DevBuf(sn.size() * sizeof(float));
    m->rope_sin.Upload(sn.data(), sn.size() * sizeof(float));
    const size_t f = sizeof(float);
    const size_t q_n = ctx * static_cast<size_t>(config->heads) * dim;
    const size_t k_n = ctx * static_cast<size_t>(config->kv_heads) * dim;
    m->hidden = DevBuf(ctx * config->hidden * f);
    m->normed = DevBuf(ctx * config->hidden * f);
    m->query = DevBuf(q_n * f);
    m->key = DevBuf(k_n * f);
    m->value = DevBuf(k_n * f);
    m->mixed = DevBuf(q_n * f);
    m->gate = DevBuf(ctx * config->intermediate * f);
    m->up = DevBuf(ctx * config->intermediate * f);
    m->logits = DevBuf(static_cast<size_t>(config->vocab) * f);
    m->chosen = DevBuf(ctx * sizeof(int32_t));
    m->prompt_ids = DevBuf(ctx * sizeof(int32_t));
    m->words = DevBuf(64);
    // Room for the chunk partials and for the fixed-split partials of the decode attention.
    m->attn_work = DevBuf(std::max(AttentionWorkBytes(1, config->heads, config->context - 1, dim),
                                   static_cast<size_t>(config->heads) * kDecodeSplitMaxBytesPerHead));
    m->attn_arrivals = DevBuf(static_cast<size_t>(config->heads) * sizeof(uint32_t));
    m->greedy_work = DevBuf(GreedyWorkBytes(config->vocab));
    m->greedy_keys = DevBuf(static_cast<size_t>((config->vocab + 7) / 8) * sizeof(uint64_t));
    for (int32_t l = 0; l < config->layers; ++l) {
      m->k_cache.emplace_back(k_n * f);
      m->v_cache.emplace_back(k_n * f);
    }
    made = m.release();
  });
  return rc == 0 ? reinterpret_cast<AccelLlama*>(made) : nullptr;
}

ACCEL_LLAMA_API void accel_llama_destroy(AccelLlama* model) {
  if (model == nullptr) return;
  accel_hip_synchronize();
  delete Get(model);
}

ACCEL_LLAMA_API int accel_llama_weight(AccelLlama* handle, int32_t kind, int32_t layer, const float* data,
                                       int64_t rows, int64_t cols) {
  Model* m = Get(handle);
  if (m == nullptr || data == nullptr || rows <= 0 || cols <= 0 || !ShapeOk(*m, kind, rows, cols)) {
    g_llama_error = "invalid weight";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    m->DropDecodeGraph();
    const size_t bytes = static_cast<size_t>(rows * cols) * sizeof(float);
    if (IsNorm(kind)) {
      DevBuf* slot = NormSlot(*m, kind, layer);
      if (slot == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "unknown weight");
      DevBuf b(bytes);
      b.Upload(data, bytes);
      *slot = std::move(b);
    } else if (kind == ACCEL_W_EMBED) {
      DevBuf b(bytes);
      b.Upload(data, bytes);
      m->embed_f = std::move(b);
      m->embed_q = DevBuf();
      m->embed_scale = DevBuf();
    } else {
      const Part p = PartOf(*m, kind, layer);
      if (p.linear == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "unknown weight");
      const std::vector<float> t = Transposed(data, rows, cols);
      UploadPart(p, false, t.data(), nullptr);
    }
  });
}

ACCEL_LLAMA_API int accel_llama_weight_q8(AccelLlama* handle, int32_t kind, int32_t layer, const int8_t* q,
                                          const float* row_scale, int64_t rows, int64_t cols) {
  Model* m = Get(handle);
  if (m == nullptr || q == nullptr || row_scale == nullptr || rows <= 0 || cols <= 0 || IsNorm(kind) ||
      !ShapeOk(*m, kind, rows, cols)) {
    g_llama_error = "invalid weight";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    m->DropDecodeGraph();
    const size_t bytes = static_cast<size_t>(rows * cols);
    const size_t sbytes = static_cast<size_t>(rows) * sizeof(float);
    if (kind == ACCEL_W_EMBED) {
      DevBuf qb(bytes), sb(sbytes);
      qb.Upload(q, bytes);
      sb.Upload(row_scale, sbytes);
      m->embed_q = std::move(qb);
      m->embed_scale = std::move(sb);
      m->embed_f = DevBuf();
      return;
    }
    const Part p = PartOf(*m, kind, layer);
    if (p.linear == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "unknown weight");
    const std::vector<int8_t> t = Transposed(q, rows, cols);
    UploadPart(p, true, t.data(), row_scale);
  });
}

ACCEL_LLAMA_API int accel_llama_generate(AccelLlama* handle, const int32_t* prompt, int32_t prompt_count,
                                         int32_t max_new, int32_t eos_id, float temperature, uint32_t seed,
                                         int32_t top_k, int32_t* out_ids, int32_t* out_count) {
  Model* m = Get(handle);
  if (m == nullptr || prompt == nullptr || out_ids == nullptr || out_count == nullptr || prompt_count <= 0 ||
      max_new < 0) {
    g_llama_error = "invalid generate";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    if (!m->Ready()) Fail(ACCEL_HIP_INVALID_ARGUMENT, "llama weights are incomplete");
    m->Generate(prompt, prompt_count, max_new, eos_id, temperature, seed, top_k, out_ids, out_count, nullptr,
                nullptr);
  });
}

ACCEL_LLAMA_API int accel_llama_tokenizer(AccelLlama* handle, const char* path) {
  Model* m = Get(handle);
  if (m == nullptr || path == nullptr || path[0] == '\0') {
    g_llama_error = "invalid tokenizer";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    m->bpe.Load(path);
  });
}

ACCEL_LLAMA_API int accel_llama_encode(AccelLlama* handle, const char* text, int32_t text_len, int32_t* out_ids,
                                       int32_t out_cap, int32_t* out_count) {
  Model* m = Get(handle);
  if (m == nullptr || text_len < 0 || (text_len > 0 && text == nullptr) || out_ids == nullptr ||
      out_count == nullptr || out_cap < 0) {
    g_llama_error = "invalid encode";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    const std::vector<int32_t> ids =
        m->bpe.Encode(text_len == 0 ? std::string_view() : std::string_view(text, static_cast<size_t>(text_len)));
    if (static_cast<int64_t>(ids.size()) > out_cap) Fail(ACCEL_HIP_INVALID_ARGUMENT, "encode buffer is too small");
    if (!ids.empty()) std::memcpy(out_ids, ids.data(), ids.size() * sizeof(int32_t));
    *out_count = static_cast<int32_t>(ids.size());
  });
}

ACCEL_LLAMA_API int accel_llama_decode(AccelLlama* handle, const int32_t* ids, int32_t count, int32_t skip_special,
                                       char* out_text, int32_t out_cap, int32_t* out_len) {
  Model* m = Get(handle);
  if (m == nullptr || out_text == nullptr || out_len == nullptr || count < 0 || (count > 0 && ids == nullptr) ||
      out_cap < 0) {
    g_llama_error = "invalid decode";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    const std::string text = m->bpe.Decode(ids, count, skip_special != 0);
    if (static_cast<int64_t>(text.size()) > out_cap) Fail(ACCEL_HIP_INVALID_ARGUMENT, "decode buffer is too small");
    if (!text.empty()) std::memcpy(out_text, text.data(), text.size());
    *out_len = static_cast<int32_t>(text.size());
  });
}

ACCEL_LLAMA_API int accel_llama_complete_stream(AccelLlama* handle, const char* prompt, int32_t prompt_len,
                                                int32_t max_new, int32_t eos_id, float temperature, uint32_t seed,
                                                int32_t top_k, char* out_text, int32_t out_text_cap,
                                                int32_t* out_text_len, int32_t* out_ids, int32_t out_ids_cap,
                                                int32_t* out_count, int32_t* prompt_tokens, AccelLlamaTokenFn on_token,
                                                void* user) {
  Model* m = Get(handle);
  if (m == nullptr || prompt_len < 0 || (prompt_len > 0 && prompt == nullptr) || max_new < 0) {
    g_llama_error = "invalid complete";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    if (!m->Ready()) Fail(ACCEL_HIP_INVALID_ARGUMENT, "llama weights are incomplete");
    m->Complete(prompt, prompt_len, max_new, eos_id, temperature, seed, top_k, out_text, out_text_cap, out_text_len,
                out_ids, out_ids_cap, out_count, prompt_tokens, on_token, user);
  });
}

ACCEL_LLAMA_API int accel_llama_complete(AccelLlama* handle, const char* prompt, int32_t prompt_len, int32_t max_new,
                                         int32_t eos_id, float temperature, uint32_t seed, int32_t top_k,
                                         char* out_text, int32_t out_text_cap, int32_t* out_text_len, int32_t* out_ids,
                                         int32_t out_ids_cap, int32_t* out_count, int32_t* prompt_tokens) {
  return accel_llama_complete_stream(handle, prompt, prompt_len, max_new, eos_id, temperature, seed, top_k, out_text,
                                     out_text_cap, out_text_len, out_ids, out_ids_cap, out_count, prompt_tokens,
                                     nullptr, nullptr);
}

ACCEL_LLAMA_API int accel_llama_forward_ids(AccelLlama* handle, const int32_t* ids, int32_t count, int32_t reset) {
  Model* m = Get(handle);
  if (m == nullptr) {
    g_llama_error = "invalid forward";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    if (!m->Ready()) Fail(ACCEL_HIP_INVALID_ARGUMENT, "llama weights are incomplete");
    if (ids == nullptr || count <= 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "invalid forward");
    if (reset) m->filled = 0;
    if (m->filled < 0 || count > m->cfg.context - m->filled) Fail(ACCEL_HIP_INVALID_ARGUMENT, "forward exceeds context");
    m->prompt_ids.Upload(ids, static_cast<size_t>(count) * sizeof(int32_t));
    m->Forward(m->prompt_ids.as<int32_t>(), count, 0, true);
    m->NoteForward();
    m->filled += count;
  });
}

ACCEL_LLAMA_API int accel_llama_logits(AccelLlama* handle, float* out, int32_t count) {
  Model* m = Get(handle);
  if (m == nullptr || out == nullptr || count != (m ? m->cfg.vocab : 0)) {
    g_llama_error = "invalid logit read";
    return 1;
  }
  return Run([&] {
    std::lock_guard<std::mutex> lock(m->mu);
    if (accel_hip_peek(out, m->logits.as<float>(), static_cast<size_t>(count) * sizeof(float)) != ACCEL_HIP_OK)
      Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
  });
}

ACCEL_LLAMA_API int accel_llama_logit_max_abs(AccelLlama* handle, const float* reference, int32_t count,
                                             float* out_max_abs) {
  Model* m = Get(handle);
  if (m == nullptr || reference == nullptr || out_max_abs == nullptr || count != m->cfg.vocab) {
    g_llama_error = "invalid logit reference";
    return 1;
  }
  return Run([&] {
    std::vector<float> row(static_cast<size_t>(count));
    {
      std::lock_guard<std::mutex> lock(m->mu);
      if (accel_hip_peek(row.data(), m->logits.as<float>(), row.size() * sizeof(float)) != ACCEL_HIP_OK)
        Fail(ACCEL_HIP_RUNTIME_ERROR, accel_hip_last_error());
    }
    float worst = 0.f;
    for (int32_t i = 0; i < count; ++i) {
      const float d = std::fabs(row[static_cast<size_t>(i)] - reference[i]);
      if (d > worst) worst = d;
    }
    *out_max_abs = worst;
  });
}

ACCEL_LLAMA_API int accel_llama_set_fused_inputs(AccelLlama* handle, int32_t enable) {
  Model* m = Get(handle);
  if (m == nullptr) {
    g_llama_error = "invalid model";
    return 1;
  }
  return Run([&] {
    if (enable < 0 || enable > 7) Fail(ACCEL_HIP_INVALID_ARGUMENT, "fused inputs: enable must be 0 .. 7");
    std::lock_guard<std::mutex> lock(m->mu);
    if (m->fuse != enable) m->DropDecodeGraph();  // the graph holds the other kernels
    m->fuse = enable;
  });
}

ACCEL_LLAMA_API void accel_llama_reset(AccelLlama* handle) {
  Model* m = Get(handle);
  if (m == nullptr) return;
  std::lock_guard<std::mutex> lock(m->mu);
  m->filled = 0;
}

ACCEL_LLAMA_API const char* accel_llama_last_error(void) { return g_llama_error.c_str(); }

}  // extern "C"

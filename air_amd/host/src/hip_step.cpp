// hip_step.cpp -- HipStepEngine and HipSequence: the Qwen2 step on one GPU.
//
// Per step the host validates the rows, reserves KV pages, uploads tokens,
// positions and page tables through one pinned staging copy, issues the
// layer loop through the air_hip C ABI on the model's stream and reads back
// only what the rows asked for (greedy ids, or logits rows).  The step
// follows ReferenceExecutor::step_impl (src/reference/reference_executor.cpp:
// 325-428) operation by operation; its validation messages are the
// reference's (reference_executor.cpp:328-335).
#include "air/hip_step.hpp"
#include "air/profile.hpp"

#include "air/synthetic.hpp"
#include "air_hip.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>

namespace air {

namespace {

Status runtime_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return Status::ok();
    return Status::internal_error(std::string(what) + ": " + hipGetErrorString(e));
}

// f32 (or f16) norm vector of `width` values, as ReferenceTensorReader::vector
// decodes it (tensor_reader.cpp:325-345).
Result<std::vector<float>> norm_vector(const ModelDefinition& model, const std::string& name, std::uint64_t width) {
    const auto* t = model.find_tensor(name);
    if (!t) return Status::data_error("missing tensor: " + name);
    if (t->shape.element_count() != width) return Status::data_error("norm width mismatch: " + name);
    auto bytes = model.tensor_bytes(*t);
    if (!bytes) return bytes.status();
    std::vector<float> out(width);
    if (t->format_type == static_cast<std::uint32_t>(GgmlType::f32) && bytes.value().size() == width * 4U) {
        std::memcpy(out.data(), bytes.value().data(), width * 4U);
    } else if (t->format_type == static_cast<std::uint32_t>(GgmlType::f16) && bytes.value().size() == width * 2U) {
        for (std::uint64_t i = 0; i < width; ++i) {
            std::uint16_t h = 0;
            std::memcpy(&h, bytes.value().data() + 2U * i, 2U);
            out[i] = f16_bits_to_f32(h);
        }
    } else {
        return Status::unsupported("norm weights must be f32 or f16: " + name);
    }
    return out;
}

} // namespace

// ---- HipSequence ------------------------------------------------------------

HipSequence::HipSequence(HipStepEngine& engine, const LinearPolicy& linear, const AttentionPolicy& attention)
    : engine_(engine),
      prefill_block_(linear.prefill_block),
      decode_block_(linear.decode_block),
      decode_output_(linear.decode_output),
      prefill_attention_(attention.prefill),
      decode_attention_(attention.decode) {}

HipSequence::~HipSequence() { engine_.release_pages(pages_); }

namespace {

std::vector<StepRow> prompt_rows(HipSequence* seq, std::span<const TokenId> tokens, RowOutput last) {
    std::vector<StepRow> rows(tokens.size());
    for (std::size_t i = 0; i < tokens.size(); ++i) rows[i] = StepRow{seq, tokens[i], RowOutput::none};
    if (!rows.empty()) rows.back().output = last;
    return rows;
}

} // namespace

// A prompt longer than the engine's step width runs as consecutive steps.
Result<std::vector<float>> HipSequence::prefill(std::span<const TokenId> tokens) {
    if (tokens.empty()) return Status::invalid_argument("prefill requires at least one token");
    std::vector<float> logits;
    const std::size_t width = engine_.max_rows();
    for (std::size_t begin = 0; begin < tokens.size(); begin += width) {
        const std::size_t count = std::min(width, tokens.size() - begin);
        const bool last = begin + count == tokens.size();
        auto rows = prompt_rows(this, tokens.subspan(begin, count), last ? RowOutput::logits : RowOutput::none);
        auto result = engine_.run(rows, prefill_block_, decode_output_, prefill_attention_);
        if (!result) return result.status();
        if (last) logits = std::move(result.value().logits.front());
    }
    return logits;
}

Status HipSequence::prefill_discard(std::span<const TokenId> tokens) {
    if (tokens.empty()) return Status::invalid_argument("prefill requires at least one token");
    const std::size_t width = engine_.max_rows();
    for (std::size_t begin = 0; begin < tokens.size(); begin += width) {
        const std::size_t count = std::min(width, tokens.size() - begin);
        auto rows = prompt_rows(this, tokens.subspan(begin, count), RowOutput::none);
        auto result = engine_.run(rows, prefill_block_, decode_output_, prefill_attention_);
        if (!result) return result.status();
    }
    return Status::ok();
}

Result<TokenId> HipSequence::prefill_greedy(std::span<const TokenId> tokens) {
    if (tokens.empty()) return Status::invalid_argument("prefill requires at least one token");
    TokenId token = 0;
    const std::size_t width = engine_.max_rows();
    for (std::size_t begin = 0; begin < tokens.size(); begin += width) {
        const std::size_t count = std::min(width, tokens.size() - begin);
        const bool last = begin + count == tokens.size();
        auto rows = prompt_rows(this, tokens.subspan(begin, count), last ? RowOutput::greedy : RowOutput::none);
        auto result = engine_.run(rows, prefill_block_, decode_output_, prefill_attention_);
        if (!result) return result.status();
        if (last) token = result.value().greedy.front();
    }
    return token;
}

Result<std::vector<float>> HipSequence::decode(TokenId token) {
    const StepRow row{this, token, RowOutput::logits};
    auto result = engine_.run({&row, 1}, decode_block_, decode_output_, decode_attention_);
    if (!result) return result.status();
    return std::move(result.value().logits.front());
}

Result<TokenId> HipSequence::decode_greedy(TokenId token) {
    const StepRow row{this, token, RowOutput::greedy};
    auto result = engine_.run({&row, 1}, decode_block_, decode_output_, decode_attention_);
    if (!result) return result.status();
    return result.value().greedy.front();
}

runtime_detail::SequenceResources HipSequence::resources() const noexcept {
    const std::uint64_t kv = static_cast<std::uint64_t>(pages_.size()) * engine_.page_bytes();
    return {tokens_, kv, kv};
}

Result<std::unique_ptr<runtime_detail::SequenceCheckpoint>> HipSequence::checkpoint() const {
    return Status::unsupported("HIP sequences do not provide checkpoints");
}

// ---- HipStepEngine ---------------------------------------------------------

Status HipStepEngine::allocate(void** ptr, std::uint64_t bytes, const char* what) {
    *ptr = nullptr;
    if (bytes == 0U) return Status::ok();
    if (Status s = runtime_status(hipMalloc(ptr, bytes), what); !s) return s;
    allocations_.push_back(*ptr);
    resident_bytes_ += bytes;
    return Status::ok();
}

HipStepEngine::~HipStepEngine() {
    (void)hipSetDevice(prepared_.device());
    (void)hipStreamSynchronize(static_cast<hipStream_t>(stream()));
    for (auto& [key, graph] : graphs_) {
        if (graph.exec) (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph.exec));
    }
    for (void* p : allocations_) (void)hipFree(p);
    for (void* p : chunks_) (void)hipFree(p);
    if (staging_) (void)hipHostFree(staging_);
    if (chunk_host_) (void)hipHostFree(chunk_host_);
    if (owns_embedding_ && embedding_) air_hip_matrix_release(embedding_);
}

std::uint64_t HipStepEngine::kv_page_bytes(const ModelConfig& c, std::uint32_t page_tokens) noexcept {
    if (c.attention_head_count == 0U) return 0U;
    const std::uint64_t kv_width = static_cast<std::uint64_t>(c.kv_head_count) * (c.embedding_size / c.attention_head_count);
    return static_cast<std::uint64_t>(c.layer_count) * 2U * page_tokens * kv_width * sizeof(float);
}

std::uint32_t HipStepEngine::planned_pool_pages(const HipPreparedModel& prepared, std::uint32_t page_tokens) {
    if (page_tokens == 0U || kv_page_bytes(prepared.model().config(), page_tokens) == 0U) return 0U;
    return prepared.options().kv_pool_pages;
}

std::uint32_t HipStepEngine::chunk_shift_for(std::uint64_t page_bytes, std::uint32_t requested) noexcept {
    std::uint64_t pages = requested;
    if (pages == 0U) pages = page_bytes ? (256ULL << 20) / page_bytes : 1U;
    pages = std::clamp<std::uint64_t>(pages, 1U, 65536U);
    std::uint32_t shift = 0;
    while ((2ULL << shift) <= pages) ++shift;
    return shift;
}

air_hip_kv_layout HipStepEngine::kv_layout(std::uint32_t table_pages) const noexcept {
    const auto& c = prepared_.model().config();
    return air_hip_kv_layout{pool_, page_tokens_, kv_width_, c.layer_count, table_pages, pool_pages_,
                             growable_ ? chunk_table_ : nullptr, growable_ ? chunk_shift_ : 0U};
}

// A growing pool takes chunks as steps need pages: each chunk is zeroed (the
// attention reads whole chunks of keys, and a slot not yet written must hold
// finite values) and its base uploaded into the device table, both on the
// engine's stream, so the step that takes its pages runs after them.  The
// pages of a new chunk go on the free list lowest id last (taken first).
Status HipStepEngine::grow_pool(std::uint64_t missing) {
    const std::uint64_t per_chunk = 1ULL << chunk_shift_;
    const auto stream_ = static_cast<hipStream_t>(stream());
    while (missing > 0U) {
        const std::size_t c = chunks_.size();
        if (c >= kMaxKvChunks) {
            return Status::invalid_state("HIP KV page pool exhausted: its chunk table holds " +
                                         std::to_string(kMaxKvChunks) + " chunks");
        }
        const std::uint64_t bytes = per_chunk * page_bytes_;
        void* chunk = nullptr;
        if (hipMalloc(&chunk, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return Status::invalid_state("HIP KV page pool exhausted: " + std::to_string(missing) +
                                         " more pages needed and no device memory for a chunk of " +
                                         std::to_string(per_chunk));
        }
        chunks_.push_back(chunk);
        chunk_host_[c] = static_cast<float*>(chunk);
        if (Status s = runtime_status(hipMemsetAsync(chunk, 0, bytes, stream_), "hipMemsetAsync(kv chunk)"); !s) {
            return s;
        }
        if (Status s = runtime_status(hipMemcpyAsync(chunk_table_ + c, chunk_host_ + c, sizeof(float*),
                                                     hipMemcpyHostToDevice, stream_),
                                      "hipMemcpyAsync(kv chunk table)");
            !s) {
            return s;
        }
        const auto first = static_cast<std::int32_t>(c * per_chunk);
        for (std::uint64_t i = per_chunk; i-- > 0U;) free_pages_.push_back(first + static_cast<std::int32_t>(i));
        allocated_pages_.fetch_add(per_chunk, std::memory_order_relaxed);
        chunk_bytes_.fetch_add(bytes, std::memory_order_relaxed);
        missing = missing > per_chunk ? missing - per_chunk : 0U;
    }
    return Status::ok();
}

Result<std::unique_ptr<HipStepEngine>> HipStepEngine::create(const HipPreparedModel& prepared,
                                                             std::uint32_t page_tokens, std::uint32_t pool_pages,
                                                             std::uint32_t max_rows) {
    const auto& model = prepared.model();
    const auto& c = model.config();
    if (page_tokens == 0U) return Status::invalid_argument("KV page size must be non-zero");
    if (max_rows == 0U || max_rows > 4096U) return Status::invalid_argument("step width must be in [1, 4096]");
    if (c.attention_head_count == 0U || c.embedding_size % c.attention_head_count != 0U) {
        return Status::data_error("embedding width must divide into the attention heads");
    }
    const std::uint32_t head_dim = c.embedding_size / c.attention_head_count;
    if (c.kv_head_count == 0U || c.attention_head_count % c.kv_head_count != 0U) {
        return Status::data_error("attention heads must be a multiple of the KV heads");
    }
    if (c.rope_dimension_count == 0U || c.rope_dimension_count > head_dim || c.rope_dimension_count % 2U != 0U) {
        return Status::invalid_state("Qwen2 reference executor requires an even RoPE dimension within each head");
    }
    if (!(c.rope_frequency_base > 0.0)) {
        return Status::invalid_state("Qwen2 reference executor requires a positive RoPE base");
    }
    if (head_dim > 512U) return Status::unsupported("HIP attention supports head widths up to 512");
    if (c.context_length == 0U || c.context_length > static_cast<std::uint64_t>(INT32_MAX)) {
        return Status::unsupported("context length must be in [1, 2^31)");
    }

    std::unique_ptr<HipStepEngine> e(new HipStepEngine(prepared));
    e->page_tokens_ = page_tokens;
    e->pool_pages_ = pool_pages;
    e->max_rows_ = max_rows;
    e->max_pages_ = static_cast<std::uint32_t>((c.context_length + page_tokens - 1U) / page_tokens);
    e->output_rows_ = std::min<std::uint32_t>(max_rows, AIR_HIP_MAX_DECODE_ROWS);
    e->embed_ = c.embedding_size;
    e->head_dim_ = head_dim;
    e->q_width_ = c.attention_head_count * head_dim;
    e->kv_width_ = c.kv_head_count * head_dim;
    e->qkv_width_ = e->q_width_ + 2U * e->kv_width_;
    e->ffn_ = c.feed_forward_size;
    e->vocab_ = c.vocabulary_size;
    e->page_bytes_ = kv_page_bytes(c, page_tokens);
    if (e->page_bytes_ == 0U) return Status::invalid_state("KV pages of zero bytes");
    if (pool_pages > static_cast<std::uint32_t>(INT32_MAX)) return Status::invalid_argument("KV pool is too large");
    e->growable_ = pool_pages == 0U;
    if (e->growable_) {
        e->chunk_shift_ = chunk_shift_for(e->page_bytes_, prepared.options().kv_chunk_pages);
        e->pool_pages_ = kMaxKvChunks << e->chunk_shift_;   // every page id the table can name
    }

    if (Status s = runtime_status(hipSetDevice(prepared.device()), "hipSetDevice"); !s) return s;
    const auto upload = [&](float** dst, const std::vector<float>& host, const char* what) -> Status {
        if (Status s = e->allocate(reinterpret_cast<void**>(dst), host.size() * sizeof(float), what); !s) return s;
        return runtime_status(hipMemcpy(*dst, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice), what);
    };

    // Norm weights.
    e->attn_norm_.assign(c.layer_count, nullptr);
    e->ffn_norm_.assign(c.layer_count, nullptr);
    for (std::uint32_t l = 0; l < c.layer_count; ++l) {
        auto attn = norm_vector(model, block_tensor_name(l, "attn_norm.weight"), c.embedding_size);
        if (!attn) return attn.status();
        if (Status s = upload(&e->attn_norm_[l], attn.value(), "hipMalloc(attn_norm)"); !s) return s;
        auto ffn = norm_vector(model, block_tensor_name(l, "ffn_norm.weight"), c.embedding_size);
        if (!ffn) return ffn.status();
        if (Status s = upload(&e->ffn_norm_[l], ffn.value(), "hipMalloc(ffn_norm)"); !s) return s;
    }
    auto out_norm = norm_vector(model, "output_norm.weight", c.embedding_size);
    if (!out_norm) return out_norm.status();
    if (Status s = upload(&e->output_norm_, out_norm.value(), "hipMalloc(output_norm)"); !s) return s;

    // RoPE table: the reference's double angle per (position, pair), rounded
    // to float cos / sin (reference_executor.cpp:53-60).  1 / pow(base, 2i/d)
    // depends on i only, so it is computed once per pair with the same
    // expression.
    {
        const std::uint32_t half = c.rope_dimension_count / 2U;
        std::vector<double> inverse(half);
        for (std::uint32_t i = 0; i < half; ++i) {
            const double exponent = (2.0 * static_cast<double>(i)) / static_cast<double>(c.rope_dimension_count);
            inverse[i] = 1.0 / std::pow(c.rope_frequency_base, exponent);
        }
        std::vector<float> table(static_cast<std::size_t>(c.context_length) * half * 2U);
        for (std::uint64_t p = 0; p < c.context_length; ++p) {
            for (std::uint32_t i = 0; i < half; ++i) {
                const double angle = static_cast<double>(p) * inverse[i];
                table[(p * half + i) * 2U] = static_cast<float>(std::cos(angle));
                table[(p * half + i) * 2U + 1U] = static_cast<float>(std::sin(angle));
            }
        }
        if (Status s = upload(&e->rope_table_, table, "hipMalloc(rope)"); !s) return s;
    }

    // Embedding rows come from the resident token_embd matrix (the output
    // matrix itself when the model ties them).
    if (prepared.output_is_embedding()) {
        e->embedding_ = prepared.output_matrix();
    } else {
        const auto* t = model.find_tensor("token_embd.weight");
        if (!t) return Status::data_error("missing tensor: token_embd.weight");
        if (t->shape.dimensions.size() != 2U || t->shape.dimensions[0] != c.embedding_size ||
            t->shape.dimensions[1] != c.vocabulary_size) {
            return Status::data_error("token_embd.weight must be {embedding, vocabulary}");
        }
        auto bytes = model.tensor_bytes(*t);
        if (!bytes) return bytes.status();
        air_hip_matrix* m = nullptr;
        const int rc = air_hip_matrix_prepare(prepared.context(), static_cast<int>(t->format_type),
                                              t->shape.dimensions[0], t->shape.dimensions[1],
                                              bytes.value().data(), bytes.value().size(), 0, &m);
        if (rc != AIR_HIP_OK) return hip_status(rc);
        e->embedding_ = m;
        e->owns_embedding_ = true;
        air_hip_matrix_desc desc{};
        if (air_hip_matrix_describe(m, &desc) == AIR_HIP_OK) e->resident_bytes_ += desc.resident_bytes;
    }

    if (e->growable_) {
        // An empty chunk table; chunks come with the steps that need pages.
        if (Status s = e->allocate(reinterpret_cast<void**>(&e->chunk_table_), kMaxKvChunks * sizeof(float*),
                                   "hipMalloc(kv chunk table)");
            !s) {
            return s;
        }
        if (Status s = runtime_status(hipMemset(e->chunk_table_, 0, kMaxKvChunks * sizeof(float*)),
                                      "hipMemset(kv chunk table)");
            !s) {
            return s;
        }
        void* mirror = nullptr;
        if (Status s = runtime_status(hipHostMalloc(&mirror, kMaxKvChunks * sizeof(float*)), "hipHostMalloc(kv chunks)");
            !s) {
            return s;
        }
        e->chunk_host_ = static_cast<float**>(mirror);
    } else {
        // A fixed pool, zeroed once.
        if (Status s = e->allocate(reinterpret_cast<void**>(&e->pool_), e->page_bytes_ * pool_pages,
                                   "hipMalloc(kv pool)");
            !s) {
            return s;
        }
        if (Status s = runtime_status(hipMemset(e->pool_, 0, e->page_bytes_ * pool_pages), "hipMemset(kv pool)");
            !s) {
            return s;
        }
        e->free_pages_.resize(pool_pages);
        for (std::uint32_t i = 0; i < pool_pages; ++i) e->free_pages_[i] = static_cast<std::int32_t>(pool_pages - 1U - i);
        e->allocated_pages_.store(pool_pages, std::memory_order_relaxed);
    }

    // Step buffers.
    const std::uint64_t rows = max_rows;
    const auto buffer = [&](float** dst, std::uint64_t floats, const char* what) {
        return e->allocate(reinterpret_cast<void**>(dst), floats * sizeof(float), what);
    };
    Status s;
    if (!(s = buffer(&e->hidden_, rows * e->embed_, "hipMalloc(hidden)"))) return s;
    if (!(s = buffer(&e->normed_, rows * e->embed_, "hipMalloc(normed)"))) return s;
    if (!(s = buffer(&e->qkv_, rows * e->qkv_width_, "hipMalloc(qkv)"))) return s;
    if (!(s = buffer(&e->att_, rows * e->q_width_, "hipMalloc(attention)"))) return s;
    if (!(s = buffer(&e->proj_, rows * e->embed_, "hipMalloc(projection)"))) return s;
    if (!(s = buffer(&e->gate_up_, rows * 2U * e->ffn_, "hipMalloc(gate_up)"))) return s;
    if (!(s = buffer(&e->act_, rows * e->ffn_, "hipMalloc(activation)"))) return s;
    if (!prepared.fused_qkv() || !prepared.fused_gate_up()) {
        const std::uint64_t widest = std::max<std::uint64_t>({e->q_width_, e->kv_width_, e->ffn_});
        if (!(s = buffer(&e->part_, rows * widest, "hipMalloc(parts)"))) return s;
    }
    if (!(s = buffer(&e->final_, static_cast<std::uint64_t>(e->output_rows_) * e->embed_, "hipMalloc(final)"))) {
        return s;
    }
    if (!(s = buffer(&e->logits_, static_cast<std::uint64_t>(e->output_rows_) * e->vocab_, "hipMalloc(logits)"))) {
        return s;
    }
    // tokens | positions | page tables | attention tiles; a tile is 4 int32.
    e->tile_capacity_ = max_rows * c.attention_head_count;
    const std::uint64_t ints = rows * (2U + e->max_pages_) + 4ULL * e->tile_capacity_;
    if (!(s = e->allocate(reinterpret_cast<void**>(&e->tokens_dev_), ints * sizeof(std::int32_t), "hipMalloc(rows)"))) {
        return s;
    }
    e->positions_dev_ = e->tokens_dev_ + rows;
    e->tables_dev_ = e->positions_dev_ + rows;
    if (!(s = e->allocate(reinterpret_cast<void**>(&e->argmax_dev_), e->output_rows_ * sizeof(std::int32_t),
                          "hipMalloc(argmax)"))) {
        return s;
    }
    void* pinned = nullptr;
    if (!(s = runtime_status(hipHostMalloc(&pinned, (ints + e->output_rows_) * sizeof(std::int32_t)),
                             "hipHostMalloc(staging)"))) {
        return s;
    }
    e->staging_ = static_cast<std::int32_t*>(pinned);
    return e;
}

std::uint64_t HipStepEngine::free_pool_bytes() const noexcept {
    std::lock_guard<std::mutex> lock(pool_mutex_);
    return static_cast<std::uint64_t>(free_pages_.size()) * page_bytes_;
}

void HipStepEngine::release_pages(std::vector<std::int32_t>& pages) {
    std::lock_guard<std::mutex> lock(pool_mutex_);
    free_pages_.insert(free_pages_.end(), pages.rbegin(), pages.rend());
    pages.clear();
}

// q|k|v (or gate|up) of `m` rows into y with row stride sum(widths): the
// fused matrix in one linear, otherwise each part into `part_` and a strided
// copy into its columns.
Status HipStepEngine::project(std::uint32_t layer, LinearRole fused, LinearRole first, LinearRole second,
                              LinearRole third, const float* x, float* y, std::uint32_t m,
                              QuantizedLinearExecutionKind tactic) {
    const bool is_fused = fused == LinearRole::attn_qkv ? prepared_.fused_qkv() : prepared_.fused_gate_up();
    if (is_fused) return prepared_.linear(layer, fused, x, y, m, tactic);
    const LinearRole parts[] = {first, second, third};
    const std::size_t count = fused == LinearRole::attn_qkv ? 3U : 2U;
    std::uint64_t widths[3] = {0, 0, 0}, total = 0;
    for (std::size_t i = 0; i < count; ++i) {
        auto info = prepared_.linear_info(layer, parts[i]);
        if (!info) return info.status();
        widths[i] = info.value().n;
        total += widths[i];
    }
    std::uint64_t offset = 0;
    for (std::size_t i = 0; i < count; ++i) {
        if (Status s = prepared_.linear(layer, parts[i], x, part_, m, tactic); !s) return s;
        const hipError_t err = hipMemcpy2DAsync(y + offset, total * sizeof(float), part_, widths[i] * sizeof(float),
                                                widths[i] * sizeof(float), m, hipMemcpyDeviceToDevice,
                                                static_cast<hipStream_t>(stream()));
        if (Status s = runtime_status(err, "hipMemcpy2DAsync(parts)"); !s) return s;
        offset += widths[i];
    }
    return Status::ok();
}

// RoPE and the KV append of layer l (unless the q|k|v linear did them),
// then attention of the step's rows over their sequences' keys (q|k|v in
// qkv_, output in att_).
Status HipStepEngine::attention(std::uint32_t l, std::uint32_t m, std::uint64_t max_tokens, std::uint32_t table_pages,
                                std::uint32_t tiles, bool rope_done) {
    const auto& c = prepared_.model().config();
    air_hip_context* ctx = prepared_.context();
    const air_hip_kv_layout kv = kv_layout(table_pages);
    const bool decode = layer_range_[4] == 'd';   // "air.decode..." (cuda_backend.cu:2202,2232)
    const ScopedRange range(decode ? "air.hip.attention_decode" : "air.hip.attention_prefill");
    int rc = AIR_HIP_OK;
    if (!rope_done) {
        rc = air_hip_rope_kv_append(ctx, &kv, qkv_, qkv_width_, m, positions_dev_, tables_dev_, l,
                                    c.attention_head_count, c.kv_head_count, head_dim_, c.rope_dimension_count,
                                    rope_table_, c.context_length);
        if (rc != AIR_HIP_OK) return hip_status(rc);
    }
    rc = tiles ? air_hip_attention_online(ctx, &kv, qkv_, qkv_width_, m, positions_dev_, tables_dev_, l,
                                          c.attention_head_count, c.kv_head_count, head_dim_,
                                          reinterpret_cast<const air_hip_attention_tile*>(tiles_dev_), tiles,
                                          max_tokens, att_)
               : air_hip_attention(ctx, &kv, qkv_, qkv_width_, m, positions_dev_, tables_dev_, l,
                                   c.attention_head_count, c.kv_head_count, head_dim_, max_tokens, att_);
    return rc == AIR_HIP_OK ? Status::ok() : hip_status(rc);
}

// Embedding through the last layer's residual for `m` uploaded rows.
// tiles > 0: the online_softmax attention over the uploaded tiles; 0: the
// baseline (reference arithmetic) attention.
Status HipStepEngine::layers(std::uint32_t m, std::uint64_t max_tokens, std::uint32_t table_pages,
                             QuantizedLinearExecutionKind tactic, std::uint32_t tiles) {
    const auto& c = prepared_.model().config();
    air_hip_context* ctx = prepared_.context();
    int rc = air_hip_matrix_rows(ctx, embedding_, tokens_dev_, m, hidden_);
    if (rc != AIR_HIP_OK) return hip_status(rc);
    // One row on the decode tactic (single-sequence decode): the attention
    // norm runs inside the q|k|v linear and both residual adds inside the o
    // and down linears, the hidden state updated in place, and the SwiGLU
    // inside gate|up.  The FFN norm stays a kernel of its own: measured at
    // M = 1 on the 7B shapes, a norm prologue in each of gate|up's 1184
    // workgroups costs more than the norm launch it saves (q|k|v 9.3 us fused
    // vs 10.3 us; o + add 6.2 vs 9.8; down + add 16.4 vs 20.0; gate|up with
    // norm and SwiGLU 34.4 vs 31.6 for norm, linear and SiLU; gate|up with
    // SwiGLU alone 29.2 vs 30.4 for linear and SiLU, in graphs).
    const bool fuse = m == 1U && tactic == QuantizedLinearExecutionKind::hip_decode && prepared_.fused_qkv() &&
                      prepared_.fused_gate_up() && prepared_.tile_formats();
    const double eps = c.rms_norm_epsilon;
    const char* layer_range = layer_range_;
    if (fuse) {
        for (std::uint32_t l = 0; l < c.layer_count; ++l) {
            const ScopedRange range(layer_range);
            if (Status s = prepared_.decode_linear_fused(l, LinearRole::attn_qkv, hidden_, qkv_, attn_norm_[l], eps,
                                                         AIR_HIP_EPILOGUE_STORE);
                !s) {
                return s;
            }
            if (Status s = attention(l, m, max_tokens, table_pages, tiles); !s) return s;
            if (Status s = prepared_.decode_linear_fused(l, LinearRole::attn_output, att_, hidden_, nullptr, 0.0,
                                                         AIR_HIP_EPILOGUE_RESIDUAL);
                !s) {
                return s;
            }
            if ((rc = air_hip_rms_norm(ctx, hidden_, ffn_norm_[l], normed_, m, embed_, eps)) != AIR_HIP_OK) {
                return hip_status(rc);
            }
            if (Status s = prepared_.decode_linear_fused(l, LinearRole::ffn_gate_up, normed_, act_, nullptr, 0.0,
                                                         AIR_HIP_EPILOGUE_SWIGLU);
                !s) {
                return s;
            }
            if (Status s = prepared_.decode_linear_fused(l, LinearRole::ffn_down, act_, hidden_, nullptr, 0.0,
                                                         AIR_HIP_EPILOGUE_RESIDUAL);
                !s) {
                return s;
            }
        }
        rc = air_hip_rms_norm(ctx, hidden_, output_norm_, normed_, m, embed_, eps);
        return rc == AIR_HIP_OK ? Status::ok() : hip_status(rc);
    }
    // Each residual add runs fused with the RMSNorm after it (the next
    // layer's attention norm, or the final norm): normed_ always holds the
    // input of the next projection.  Decode widths up to 64 hand the add +
    // norm and the SwiGLU to the linear itself (air_hip_linear_epilogue),
    // whose split reduction carries them: measured on the 7B shapes at
    // M = 30 that saves three launches of 4-5 us per layer.  Prefill steps
    // hand the add + norm to o's reduction (its GEMM splits K two ways;
    // measured at M = 512: 45.9 us against 46.8 for the reduction and the
    // norm).  A row per workgroup summing down's eight splits, or q|k|v's
    // two for the RoPE and the KV append, is slower than the wide reduction
    // and the separate kernel (down 125.9 vs 121.1 us, RoPE 18.4 vs 15.6),
    // and the SwiGLU would need a context buffer as large as the step's
    // gate|up rows; those stay separate.
    const bool epilogues = tactic == QuantizedLinearExecutionKind::hip_decode && m <= AIR_HIP_MAX_DECODE_ROWS;
    // Prefill steps: the norms and the SwiGLU also leave the next prefill
    // linear's f16 operand (air_hip_rms_norm_prefill, air_hip_silu_mul_prefill),
    // so q|k|v, gate|up and down skip their conversion pass.
    const bool prefill_operands = tactic == QuantizedLinearExecutionKind::hip_prefill;
    const auto norm = [&](float* x, const float* y, const float* w, bool next_prefill) {
        if (prefill_operands && next_prefill) return air_hip_rms_norm_prefill(ctx, x, y, w, normed_, m, embed_, eps);
        return y ? air_hip_add_rms_norm(ctx, x, y, w, normed_, m, embed_, eps)
                 : air_hip_rms_norm(ctx, x, w, normed_, m, embed_, eps);
    };
    if ((rc = norm(hidden_, nullptr, attn_norm_[0], true)) != AIR_HIP_OK) {
        return hip_status(rc);
    }
    for (std::uint32_t l = 0; l < c.layer_count; ++l) {
        const ScopedRange range(layer_range);
        if (epilogues && prepared_.fused_qkv()) {
            const air_hip_kv_layout kv = kv_layout(table_pages);
            if (Status s = prepared_.linear_rope_kv(l, LinearRole::attn_qkv, normed_, m, qkv_, &kv, positions_dev_,
                                                    tables_dev_, c.attention_head_count, c.kv_head_count, head_dim_,
                                                    c.rope_dimension_count, rope_table_, c.context_length, tactic);
                !s) {
                return s;
            }
            if (Status s = attention(l, m, max_tokens, table_pages, tiles, true); !s) return s;
        } else {
            if (Status s = project(l, LinearRole::attn_qkv, LinearRole::attn_q, LinearRole::attn_k,
                                   LinearRole::attn_v, normed_, qkv_, m, tactic);
                !s) {
                return s;
            }
            if (Status s = attention(l, m, max_tokens, table_pages, tiles); !s) return s;
        }
        if (epilogues) {
            // With a fused gate|up next, the FFN norm's output is also split
            // for it (no split launch of its own).
            const int o_epilogue = m >= 2U && prepared_.fused_gate_up() ? AIR_HIP_EPILOGUE_RESIDUAL_LOAD
                                                                        : AIR_HIP_EPILOGUE_RESIDUAL;
            if (Status s = prepared_.linear_epilogue(l, LinearRole::attn_output, att_, m, hidden_, o_epilogue,
                                                     ffn_norm_[l], normed_, eps, tactic);
                !s) {
                return s;
            }
        } else if (prefill_operands) {
            // Prefill: o's K-split reduction does the residual add and the
            // norm, and leaves gate|up's f16 operand.
            if (Status s = prepared_.linear_epilogue(l, LinearRole::attn_output, att_, m, hidden_,
                                                     AIR_HIP_EPILOGUE_RESIDUAL_PREFILL, ffn_norm_[l], normed_, eps,
                                                     tactic);
                !s) {
                return s;
            }
        } else {
            if (Status s = prepared_.linear(l, LinearRole::attn_output, att_, proj_, m, tactic); !s) return s;
            if ((rc = norm(hidden_, proj_, ffn_norm_[l], true)) != AIR_HIP_OK) {
                return hip_status(rc);
            }
        }
        if (epilogues && prepared_.fused_gate_up()) {
            if (Status s = prepared_.linear_epilogue(l, LinearRole::ffn_gate_up, normed_, m, act_,
                                                     AIR_HIP_EPILOGUE_SWIGLU, nullptr, nullptr, 0.0, tactic);
                !s) {
                return s;
            }
        } else {
            if (Status s = project(l, LinearRole::ffn_gate_up, LinearRole::ffn_gate, LinearRole::ffn_up,
                                   LinearRole::ffn_up, normed_, gate_up_, m, tactic);
                !s) {
                return s;
            }
            rc = prefill_operands ? air_hip_silu_mul_prefill(ctx, gate_up_, act_, m, ffn_)
                                  : air_hip_silu_mul(ctx, gate_up_, act_, m, ffn_);
            if (rc != AIR_HIP_OK) return hip_status(rc);
        }
        const float* next_norm = l + 1U < c.layer_count ? attn_norm_[l + 1U] : output_norm_;
        if (epilogues) {
            // The next norm's output is split for its consumer too (the next
            // layer's q|k|v, or the lm_head): the split route, which Q8_0
            // q|k|v takes above 16 rows and the lm_head above 4, then needs
            // no split launch of its own.
            const int down_epilogue = m >= 2U ? AIR_HIP_EPILOGUE_RESIDUAL_LOAD : AIR_HIP_EPILOGUE_RESIDUAL;
            if (Status s = prepared_.linear_epilogue(l, LinearRole::ffn_down, act_, m, hidden_, down_epilogue,
                                                     next_norm, normed_, eps, tactic);
                !s) {
                return s;
            }
        } else {
            if (Status s = prepared_.linear(l, LinearRole::ffn_down, act_, proj_, m, tactic); !s) return s;
            if ((rc = norm(hidden_, proj_, next_norm, l + 1U < c.layer_count)) != AIR_HIP_OK) {
                return hip_status(rc);
            }
        }
    }
    return Status::ok();
}

std::uint64_t HipStepEngine::context_generation() const noexcept {
    air_hip_stats stats{};
    return air_hip_context_stats(prepared_.context(), &stats) == AIR_HIP_OK ? stats.workspace_generation : ~0ULL;
}

Status HipStepEngine::decode_device(std::uint32_t m, std::uint64_t max_tokens, std::uint32_t table_pages,
                                    QuantizedLinearExecutionKind block, QuantizedLinearExecutionKind output,
                                    std::uint32_t tiles) {
    if (Status s = layers(m, max_tokens, table_pages, block, tiles); !s) return s;
    {
        const ScopedRange range(m == 1U ? "air.decode.output_projection" : "air.decode.batch.output_projection");
        if (Status s = prepared_.linear(0, LinearRole::output, normed_, logits_, m, output); !s) return s;
    }
    const ScopedRange range("air.hip.greedy_select");
    return hip_status(air_hip_argmax(prepared_.context(), logits_, m, vocab_, argmax_dev_));
}

Status HipStepEngine::decode_graph(std::uint32_t m, std::uint64_t max_tokens, std::uint32_t table_pages,
                                   QuantizedLinearExecutionKind block, QuantizedLinearExecutionKind output,
                                   std::uint32_t tiles) {
    auto* hs = static_cast<hipStream_t>(stream());
    const std::uint64_t key = (static_cast<std::uint64_t>(m) << 32) | (static_cast<std::uint64_t>(block) << 16) |
                              (static_cast<std::uint64_t>(output) << 8) | (tiles ? 1U : 0U);
    auto it = graphs_.find(key);
    if (it != graphs_.end()) {
        if (!it->second.exec) return decode_device(m, max_tokens, table_pages, block, output, tiles);
        if (it->second.generation == context_generation()) {
            return runtime_status(hipGraphLaunch(static_cast<hipGraphExec_t>(it->second.exec), hs), "hipGraphLaunch");
        }
        (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(it->second.exec));
        graphs_.erase(it);
    }
    // This step runs eagerly (growing any buffer it needs); its launches are
    // then recorded, unexecuted, for the next steps of this width.
    if (Status s = decode_device(m, max_tokens, table_pages, block, output, tiles); !s) return s;
    const std::uint64_t generation = context_generation();
    DecodeGraph entry;
    if (hipStreamBeginCapture(hs, hipStreamCaptureModeThreadLocal) == hipSuccess) {
        const Status recorded = decode_device(m, max_tokens, table_pages, block, output, tiles);
        hipGraph_t graph = nullptr;
        const hipError_t ended = hipStreamEndCapture(hs, &graph);
        hipGraphExec_t exec = nullptr;
        if (recorded && ended == hipSuccess && graph &&
            hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess &&
            context_generation() == generation) {
            entry.exec = exec;
            entry.generation = generation;
        } else if (exec) {
            (void)hipGraphExecDestroy(exec);
        }
        if (graph) (void)hipGraphDestroy(graph);
    }
    (void)hipGetLastError();  // a refused capture leaves no error behind for the next launch check
    graphs_[key] = entry;
    return Status::ok();
}

Result<StepResult> HipStepEngine::run(std::span<const StepRow> rows, QuantizedLinearExecutionKind block_tactic,
                                      QuantizedLinearExecutionKind output_tactic, AttentionExecutionKind attention) {
    const auto& c = prepared_.model().config();
    if (rows.empty()) return Status::invalid_argument("a step needs at least one row");
    if (rows.size() > max_rows_) {
        return Status::invalid_argument("step of " + std::to_string(rows.size()) + " rows exceeds the engine width " +
                                        std::to_string(max_rows_));
    }
    const auto m = static_cast<std::uint32_t>(rows.size());

    // Positions: each sequence's next tokens in row order.
    struct Claim {
        HipSequence* sequence;
        std::uint64_t rows;
        std::size_t pages_before;
    };
    std::vector<Claim> claims;
    std::vector<std::uint64_t> positions(m);
    std::vector<std::size_t> claim_of(m);
    for (std::uint32_t r = 0; r < m; ++r) {
        HipSequence* seq = rows[r].sequence;
        if (!seq || &seq->engine_ != this) return Status::invalid_argument("row belongs to another engine");
        const TokenId token = rows[r].token;
        if (token < 0 || static_cast<std::uint64_t>(token) >= c.vocabulary_size) {
            return Status::invalid_argument("input token is outside model vocabulary");
        }
        auto it = std::find_if(claims.begin(), claims.end(), [&](const Claim& x) { return x.sequence == seq; });
        if (it == claims.end()) {
            claims.push_back({seq, 0U, seq->pages_.size()});
            it = claims.end() - 1;
        }
        positions[r] = seq->tokens_ + it->rows;
        if (positions[r] >= c.context_length) return Status::invalid_state("model context length exceeded");
        ++it->rows;
        claim_of[r] = static_cast<std::size_t>(it - claims.begin());
    }

    // Pages for the new tokens; returned on any failure below.
    const auto rollback = [&]() {
        std::lock_guard<std::mutex> lock(pool_mutex_);
        for (auto& claim : claims) {
            auto& pages = claim.sequence->pages_;
            while (pages.size() > claim.pages_before) {
                free_pages_.push_back(pages.back());
                pages.pop_back();
            }
        }
    };
    std::uint32_t table_pages = 1U;
    {
        std::lock_guard<std::mutex> lock(pool_mutex_);
        std::uint64_t needed = 0;
        for (const auto& claim : claims) {
            const std::uint64_t pages = (claim.sequence->tokens_ + claim.rows + page_tokens_ - 1U) / page_tokens_;
            needed += pages - std::min<std::uint64_t>(pages, claim.sequence->pages_.size());
            table_pages = std::max<std::uint32_t>(table_pages, static_cast<std::uint32_t>(pages));
        }
        if (needed > free_pages_.size() && growable_) {
            if (Status s = grow_pool(needed - free_pages_.size()); !s) return s;
        }
        if (needed > free_pages_.size()) {
            return Status::invalid_state("HIP KV page pool exhausted: " + std::to_string(needed) + " pages needed, " +
                                         std::to_string(free_pages_.size()) + " free");
        }
        for (auto& claim : claims) {
            const std::uint64_t pages = (claim.sequence->tokens_ + claim.rows + page_tokens_ - 1U) / page_tokens_;
            while (claim.sequence->pages_.size() < pages) {
                claim.sequence->pages_.push_back(free_pages_.back());
                free_pages_.pop_back();
            }
        }
    }

    // Decode-shaped steps (one row per sequence, every row an output: greedy
    // or logits) go through a graph captured per width: their page tables
    // span the whole context and the attention is sized for it, so one graph
    // serves every step of that width.  The graph runs the lm_head and the
    // argmax over every row; logits rows are read back from its output.
    bool decode_shape = prepared_.options().decode_graphs && claims.size() == m && m <= output_rows_;
    for (std::uint32_t r = 0; r < m && decode_shape; ++r) decode_shape = rows[r].output != RowOutput::none;
    if (decode_shape) table_pages = max_pages_;

    // Upload: tokens | positions | page tables [m][table_pages], one copy.
    std::int32_t* host = staging_;
    std::uint64_t max_tokens = decode_shape ? c.context_length : 1U;
    for (std::uint32_t r = 0; r < m; ++r) {
        host[r] = rows[r].token;
        host[m + r] = static_cast<std::int32_t>(positions[r]);
        max_tokens = std::max<std::uint64_t>(max_tokens, positions[r] + 1U);
        const auto& pages = claims[claim_of[r]].sequence->pages_;
        std::int32_t* table = host + 2U * m + static_cast<std::uint64_t>(r) * table_pages;
        for (std::uint32_t p = 0; p < table_pages; ++p) table[p] = p < pages.size() ? pages[p] : -1;
    }
    // Online attention: tiles from the runs of consecutive rows of one sequence.
    std::uint32_t tiles = 0;
    std::uint64_t upload_ints = 2U * m + static_cast<std::uint64_t>(m) * table_pages;
    if (attention == AttentionExecutionKind::online_softmax) {
        std::vector<std::uint32_t> runs;
        for (std::uint32_t r = 0; r < m; ++r) {
            if (r > 0 && rows[r].sequence == rows[r - 1].sequence) {
                ++runs.back();
            } else {
                runs.push_back(1U);
            }
        }
        auto* tile_host = reinterpret_cast<air_hip_attention_tile*>(host + upload_ints);
        const int rc = air_hip_attention_make_tiles(runs.data(), static_cast<std::uint32_t>(runs.size()),
                                                    c.attention_head_count, c.kv_head_count, tile_host,
                                                    tile_capacity_, &tiles);
        if (rc != AIR_HIP_OK) {
            rollback();
            return hip_status(rc);
        }
        tiles_dev_ = tokens_dev_ + upload_ints;
        upload_ints += 4ULL * tiles;
    }
    // Device arrays are packed the same way as the host staging.
    auto* hs = static_cast<hipStream_t>(stream());
    if (Status s = runtime_status(hipSetDevice(prepared_.device()), "hipSetDevice"); !s) {
        rollback();
        return s;
    }
    std::int32_t* positions_dev = tokens_dev_ + m;
    std::int32_t* tables_dev = tokens_dev_ + 2U * m;
    if (Status s = runtime_status(hipMemcpyAsync(tokens_dev_, host, upload_ints * sizeof(std::int32_t),
                                                 hipMemcpyHostToDevice, hs),
                                  "hipMemcpyAsync(rows)");
        !s) {
        rollback();
        return s;
    }
    positions_dev_ = positions_dev;
    tables_dev_ = tables_dev;

    // The reference's stage names (cuda_backend.cu:2678,2894,3099,3253).
    layer_range_ = decode_shape ? (m == 1U ? "air.decode.layer" : "air.decode.batch.layer")
                                : (claims.size() > 1U ? "air.prefill.multi_sequence.layer" : "air.prefill.layer");
    Status status;
    {
        const ScopedRange range(decode_shape ? (m == 1U ? "air.decode.step" : "air.decode.batch")
                                             : (claims.size() > 1U ? "air.prefill.multi_sequence" : "air.prefill.chunk"));
        status = decode_shape ? decode_graph(m, max_tokens, table_pages, block_tactic, output_tactic, tiles)
                              : layers(m, max_tokens, table_pages, block_tactic, tiles);
    }

    // Output rows: lm_head (+bias) over their final-normed rows, argmax, in
    // chunks of the logits buffer.
    StepResult result;
    std::vector<std::uint32_t> outputs;
    for (std::uint32_t r = 0; r < m; ++r) {
        if (rows[r].output != RowOutput::none) outputs.push_back(r);
    }
    air_hip_context* ctx = prepared_.context();
    std::int32_t* argmax_host = staging_ + upload_ints;
    for (std::size_t begin = 0; status && begin < outputs.size(); begin += output_rows_) {
        const auto k = static_cast<std::uint32_t>(std::min<std::size_t>(output_rows_, outputs.size() - begin));
        // The chunk's rows as one block: in place when they are consecutive,
        // else gathered into final_ (runs of consecutive rows in one copy).
        const float* x = normed_ + static_cast<std::uint64_t>(outputs[begin]) * embed_;
        if (outputs[begin + k - 1] - outputs[begin] != k - 1 || reinterpret_cast<std::uintptr_t>(x) % 16U != 0) {
            for (std::uint32_t j = 0; j < k && status;) {
                std::uint32_t run = 1;
                while (j + run < k && outputs[begin + j + run] == outputs[begin + j] + run) ++run;
                status = runtime_status(hipMemcpyAsync(final_ + static_cast<std::uint64_t>(j) * embed_,
                                                       normed_ + static_cast<std::uint64_t>(outputs[begin + j]) * embed_,
                                                       static_cast<std::uint64_t>(run) * embed_ * sizeof(float),
                                                       hipMemcpyDeviceToDevice, hs),
                                        "hipMemcpyAsync(gather)");
                j += run;
            }
            x = final_;
        }
        if (!status) break;
        if (!decode_shape) {  // a decode-shaped step has its logits and argmax already
            const ScopedRange range(claims.size() > 1U ? "air.prefill.multi_sequence.output_projection"
                                                       : "air.prefill.output_projection");
            if (!(status = prepared_.linear(0, LinearRole::output, x, logits_, k, output_tactic))) break;
            if (const int rc = air_hip_argmax(ctx, logits_, k, vocab_, argmax_dev_); rc != AIR_HIP_OK) {
                status = hip_status(rc);
                break;
            }
        }
        if (!(status = runtime_status(hipMemcpyAsync(argmax_host, argmax_dev_, k * sizeof(std::int32_t),
                                                     hipMemcpyDeviceToHost, hs),
                                      "hipMemcpyAsync(argmax)"))) {
            break;
        }
        const ScopedRange readback("air.hip.logit_readback");
        std::vector<std::vector<float>> logits;
        for (std::uint32_t j = 0; j < k && status; ++j) {
            if (rows[outputs[begin + j]].output != RowOutput::logits) continue;
            logits.emplace_back(vocab_);
            status = runtime_status(hipMemcpyAsync(logits.back().data(), logits_ + static_cast<std::uint64_t>(j) * vocab_,
                                                   vocab_ * sizeof(float), hipMemcpyDeviceToHost, hs),
                                    "hipMemcpyAsync(logits)");
        }
        if (!status) break;
        if (!(status = runtime_status(hipStreamSynchronize(hs), "hipStreamSynchronize"))) break;
        // Non-finite logits fail the step, as the reference executor's
        // device flag and readback check do (cuda_backend.cu:613-624,
        // 2331, 2368): the argmax marks such a row with -1.
        for (std::uint32_t j = 0; j < k && status; ++j) {
            if (rows[outputs[begin + j]].output != RowOutput::greedy) continue;
            if (argmax_host[j] < 0) {
                status = Status::internal_error("HIP executor produced non-finite logits");
            } else {
                result.greedy.push_back(argmax_host[j]);
            }
        }
        for (auto& row : logits) {
            if (!std::all_of(row.begin(), row.end(), [](float v) { return std::isfinite(v); })) {
                status = Status::internal_error("HIP executor produced non-finite logits");
            }
            result.logits.push_back(std::move(row));
        }
        if (!status) break;
    }
    // Always drain the stream: the staging buffer is reused by the next step.
    const Status drained = runtime_status(hipStreamSynchronize(hs), "hipStreamSynchronize");
    if (status) status = drained;
    if (!status) {
        rollback();
        return status;
    }
    for (const auto& claim : claims) claim.sequence->tokens_ += claim.rows;
    return result;
}

} // namespace air

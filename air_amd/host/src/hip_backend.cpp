// hip_backend.cpp -- HipPreparedModel over the air_hip C ABI.
//
// Residency replaces the per-tensor arena upload of the CUDA executor
// (src/cuda/cuda_backend.cu:1790-1822) with one repacked matrix per
// projection; capability and byte accounting follow CudaPreparedModel
// (src/runtime/backend.cpp:268-306, 511-560), with device memory read from
// hipMemGetInfo through air_hip_mem_info.
#include "air/hip_backend.hpp"
#include "air/hip_step.hpp"

#include "air_hip.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <limits>

namespace air {

Status hip_status(int rc) {
    const std::string message = air_hip_last_error();
    switch (rc) {
    case AIR_HIP_OK: return Status::ok();
    case AIR_HIP_INVALID_ARGUMENT: return Status::invalid_argument(message);
    case AIR_HIP_INVALID_STATE: return Status::invalid_state(message);
    case AIR_HIP_IO_ERROR: return Status::io_error(message);
    case AIR_HIP_CANCELLED: return Status::cancelled(message);
    case AIR_HIP_DATA_ERROR: return Status::data_error(message);
    case AIR_HIP_UNSUPPORTED: return Status::unsupported(message);
    default: return Status::internal_error(message.empty() ? "HIP linear engine failure" : message);
    }
}

const char* to_string(LinearRole role) noexcept {
    switch (role) {
    case LinearRole::attn_qkv: return "attn_qkv";
    case LinearRole::attn_q: return "attn_q";
    case LinearRole::attn_k: return "attn_k";
    case LinearRole::attn_v: return "attn_v";
    case LinearRole::attn_output: return "attn_output";
    case LinearRole::ffn_gate_up: return "ffn_gate_up";
    case LinearRole::ffn_gate: return "ffn_gate";
    case LinearRole::ffn_up: return "ffn_up";
    case LinearRole::ffn_down: return "ffn_down";
    case LinearRole::output: return "output";
    }
    return "unknown";
}

namespace {

Status runtime_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return Status::ok();
    return Status::internal_error(std::string(what) + ": " + hipGetErrorString(e));
}

bool same_format(std::span<const TensorDescriptor* const> parts) {
    for (const auto* p : parts) {
        if (p->format_type != parts.front()->format_type) return false;
    }
    return true;
}

} // namespace

HipPreparedModel::HipPreparedModel(std::shared_ptr<const ModelDefinition> model, int device)
    : model_(std::move(model)), device_(device) {
    capabilities_.backend = BackendKind::hip;
    capabilities_.prefill_execution = PrefillExecutionKind::native_batch;
    capabilities_.kv_storage = KvStorageKind::paged;
    capabilities_.max_prefill_batch_width = 512U;
    capabilities_.max_decode_batch_width = AIR_HIP_MAX_DECODE_ROWS;
    capabilities_.sequence_checkpointing = false;
    capabilities_.exact_prefix_reuse = false;
    capabilities_.device_greedy_selection = true;
    // Tactics per scope, each naming real device work: the exact-code decode
    // linear serves every width; the f16 MFMA GEMM serves prefill blocks.
    capabilities_.prefill_block_quantized_linear = {QuantizedLinearExecutionKind::hip_decode,
                                                    QuantizedLinearExecutionKind::hip_prefill};
    capabilities_.decode_block_quantized_linear = {QuantizedLinearExecutionKind::hip_decode};
    capabilities_.decode_output_quantized_linear = {QuantizedLinearExecutionKind::hip_decode};
    // baseline: the reference executor's double-precision softmax; online:
    // the tiled f32 online-softmax kernel.
    capabilities_.prefill_attention = {AttentionExecutionKind::baseline, AttentionExecutionKind::online_softmax};
    capabilities_.decode_attention = {AttentionExecutionKind::baseline, AttentionExecutionKind::online_softmax};
}

HipPreparedModel::~HipPreparedModel() {
    engine_.reset();  // its buffers and embedding live on this model's context
    for (auto& layer : layers_) {
        for (Linear* l : {&layer.qkv, &layer.q, &layer.k, &layer.v, &layer.o, &layer.gate_up, &layer.gate, &layer.up,
                          &layer.down}) {
            release(*l);
        }
    }
    release(output_);
    if (ctx_) air_hip_context_destroy(ctx_);
    if (owned_stream_) {
        (void)hipSetDevice(device_);
        (void)hipStreamDestroy(static_cast<hipStream_t>(owned_stream_));
    }
}

void HipPreparedModel::release(Linear& linear) noexcept {
    if (linear.matrix) air_hip_matrix_release(linear.matrix);
    if (linear.bias) {
        (void)hipSetDevice(device_);
        (void)hipFree(linear.bias);
    }
    linear = Linear{};
}

Status HipPreparedModel::make_linear(std::span<const TensorDescriptor* const> parts,
                                     std::span<const TensorDescriptor* const> biases, Linear& out) {
    const auto* first = parts.front();
    if (first->shape.dimensions.size() != 2U) return Status::data_error("linear weight must be rank 2: " + first->name);
    const std::uint64_t k = first->shape.dimensions[0];
    std::uint64_t n = 0;
    for (const auto* p : parts) {
        if (p->format_type != first->format_type || p->shape.dimensions.size() != 2U || p->shape.dimensions[0] != k) {
            return Status::data_error("fused linear parts disagree in format or input width: " + p->name);
        }
        n += p->shape.dimensions[1];
    }

    std::vector<std::byte> joined;
    std::span<const std::byte> canonical;
    if (parts.size() == 1U) {
        auto bytes = model_->tensor_bytes(*first);
        if (!bytes) return bytes.status();
        canonical = bytes.value();
    } else {
        for (const auto* p : parts) {
            auto bytes = model_->tensor_bytes(*p);
            if (!bytes) return bytes.status();
            joined.insert(joined.end(), bytes.value().begin(), bytes.value().end());
        }
        canonical = joined;
    }
    air_hip_matrix* matrix = nullptr;
    const int rc = air_hip_matrix_prepare(ctx_, static_cast<int>(first->format_type), k, n, canonical.data(),
                                          canonical.size(), 0, &matrix);
    if (rc != AIR_HIP_OK) return hip_status(rc);
    out.matrix = matrix;
    air_hip_matrix_desc desc{};
    if (const int d = air_hip_matrix_describe(matrix, &desc); d != AIR_HIP_OK) return hip_status(d);
    out.info = HipLinearInfo{first->format_type, k, n, false, desc.resident_bytes};

    // Biases: f32 per part; an absent part bias contributes zeros.
    if (std::none_of(biases.begin(), biases.end(), [](const TensorDescriptor* b) { return b != nullptr; })) {
        return Status::ok();
    }
    std::vector<float> bias(n, 0.0f);
    std::uint64_t offset = 0;
    for (std::size_t i = 0; i < parts.size(); ++i) {
        const auto width = parts[i]->shape.dimensions[1];
        if (const auto* b = biases[i]) {
            if (b->format_type != static_cast<std::uint32_t>(GgmlType::f32) || b->byte_size != width * sizeof(float)) {
                return Status::unsupported("linear bias must be f32 of the output width: " + b->name);
            }
            auto bytes = model_->tensor_bytes(*b);
            if (!bytes) return bytes.status();
            std::memcpy(bias.data() + offset, bytes.value().data(), bytes.value().size());
        }
        offset += width;
    }
    Status s = runtime_status(hipSetDevice(device_), "hipSetDevice");
    if (!s) return s;
    void* device_bias = nullptr;
    if (!(s = runtime_status(hipMalloc(&device_bias, n * sizeof(float)), "hipMalloc(bias)"))) return s;
    out.bias = static_cast<float*>(device_bias);
    if (!(s = runtime_status(hipMemcpy(device_bias, bias.data(), n * sizeof(float), hipMemcpyHostToDevice),
                             "hipMemcpy(bias)"))) {
        return s;
    }
    out.info.has_bias = true;
    bias_bytes_ += n * sizeof(float);
    return Status::ok();
}

Result<std::unique_ptr<HipPreparedModel>> HipPreparedModel::create(std::shared_ptr<const ModelDefinition> model,
                                                                   const HipPrepareOptions& options) {
    if (!model) return Status::invalid_argument("HIP backend requires a model");
    if (Status s = model->validate(); !s) return s;
    if (Status s = validate_qwen2_structure(*model); !s) return s;
    if (options.max_decode_rows == 0U || options.max_decode_rows > AIR_HIP_MAX_DECODE_ROWS) {
        return Status::invalid_argument("max_decode_rows must be in [1, 64]");
    }

    std::unique_ptr<HipPreparedModel> prepared(new HipPreparedModel(model, options.device));
    prepared->options_ = options;
    if (!options.stream) {
        // A stream of the model's own (default priority): the legacy stream
        // cannot be captured into graphs.
        if (Status s = runtime_status(hipSetDevice(options.device), "hipSetDevice"); !s) return s;
        hipStream_t stream = nullptr;
        if (Status s = runtime_status(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate"); !s) {
            return s;
        }
        prepared->owned_stream_ = stream;
        prepared->options_.stream = stream;
    }
    if (const int rc = air_hip_context_create(options.device, prepared->options_.stream, &prepared->ctx_);
        rc != AIR_HIP_OK) {
        return hip_status(rc);
    }
    const auto& c = model->config();
    const std::uint64_t head = c.embedding_size / c.attention_head_count;
    const std::uint64_t max_k = std::max<std::uint64_t>({c.embedding_size, c.feed_forward_size,
                                                         static_cast<std::uint64_t>(c.attention_head_count) * head});
    if (const int rc = air_hip_context_reserve(prepared->ctx_, max_k, options.max_decode_rows); rc != AIR_HIP_OK) {
        return hip_status(rc);
    }

    const auto tensor = [&](std::uint32_t layer, const char* suffix) {
        return model->find_tensor(block_tensor_name(layer, suffix));
    };
    prepared->layers_.resize(c.layer_count);
    bool fused_qkv = options.fuse;
    bool fused_gate_up = options.fuse;
    for (std::uint32_t l = 0; l < c.layer_count; ++l) {
        const TensorDescriptor* qkv[] = {tensor(l, "attn_q.weight"), tensor(l, "attn_k.weight"),
                                         tensor(l, "attn_v.weight")};
        const TensorDescriptor* gate_up[] = {tensor(l, "ffn_gate.weight"), tensor(l, "ffn_up.weight")};
        fused_qkv = fused_qkv && same_format(qkv);
        fused_gate_up = fused_gate_up && same_format(gate_up);
        const TensorDescriptor* linears[] = {qkv[0], qkv[1], qkv[2], gate_up[0], gate_up[1],
                                             tensor(l, "attn_output.weight"), tensor(l, "ffn_down.weight")};
        for (const TensorDescriptor* t : linears) {
            const int type = t ? static_cast<int>(t->format_type) : -1;
            if (type != AIR_HIP_TYPE_Q8_0 && type != AIR_HIP_TYPE_Q5_0 && type != AIR_HIP_TYPE_Q4_0 &&
                type != AIR_HIP_TYPE_Q4_K) {
                prepared->tile_formats_ = false;
            }
        }
    }
    prepared->fused_qkv_ = fused_qkv;
    prepared->fused_gate_up_ = fused_gate_up;

    const TensorDescriptor* none[] = {nullptr, nullptr, nullptr};
    for (std::uint32_t l = 0; l < c.layer_count; ++l) {
        auto& layer = prepared->layers_[l];
        const TensorDescriptor* qkv[] = {tensor(l, "attn_q.weight"), tensor(l, "attn_k.weight"),
                                         tensor(l, "attn_v.weight")};
        const TensorDescriptor* qkv_bias[] = {tensor(l, "attn_q.bias"), tensor(l, "attn_k.bias"),
                                              tensor(l, "attn_v.bias")};
        Status s;
        if (fused_qkv) {
            s = prepared->make_linear(qkv, qkv_bias, layer.qkv);
        } else {
            Linear* dst[] = {&layer.q, &layer.k, &layer.v};
            for (int i = 0; i < 3 && s; ++i) {
                s = prepared->make_linear({&qkv[i], 1}, {&qkv_bias[i], 1}, *dst[i]);
            }
        }
        if (!s) return s;
        const TensorDescriptor* o[] = {tensor(l, "attn_output.weight")};
        if (!(s = prepared->make_linear(o, {none, 1}, layer.o))) return s;
        const TensorDescriptor* gate_up[] = {tensor(l, "ffn_gate.weight"), tensor(l, "ffn_up.weight")};
        if (fused_gate_up) {
            s = prepared->make_linear(gate_up, {none, 2}, layer.gate_up);
        } else {
            s = prepared->make_linear({&gate_up[0], 1}, {none, 1}, layer.gate);
            if (s) s = prepared->make_linear({&gate_up[1], 1}, {none, 1}, layer.up);
        }
        if (!s) return s;
        const TensorDescriptor* down[] = {tensor(l, "ffn_down.weight")};
        if (!(s = prepared->make_linear(down, {none, 1}, layer.down))) return s;
    }
    const TensorDescriptor* out[] = {model->find_tensor("output.weight")};
    if (!out[0]) {
        out[0] = model->find_tensor("token_embd.weight");  // tied embeddings
        prepared->output_is_embedding_ = true;
    }
    const TensorDescriptor* out_bias[] = {model->find_tensor("output.bias")};
    if (Status s = prepared->make_linear(out, out_bias, prepared->output_); !s) return s;
    if (Status s = prepared->synchronize(); !s) return s;
    return prepared;
}

const HipPreparedModel::Linear* HipPreparedModel::find(std::uint32_t layer, LinearRole role) const noexcept {
    if (role == LinearRole::output) return &output_;
    if (layer >= layers_.size()) return nullptr;
    const auto& l = layers_[layer];
    const Linear* p = nullptr;
    switch (role) {
    case LinearRole::attn_qkv: p = &l.qkv; break;
    case LinearRole::attn_q: p = &l.q; break;
    case LinearRole::attn_k: p = &l.k; break;
    case LinearRole::attn_v: p = &l.v; break;
    case LinearRole::attn_output: p = &l.o; break;
    case LinearRole::ffn_gate_up: p = &l.gate_up; break;
    case LinearRole::ffn_gate: p = &l.gate; break;
    case LinearRole::ffn_up: p = &l.up; break;
    case LinearRole::ffn_down: p = &l.down; break;
    case LinearRole::output: break;
    }
    return p && p->matrix ? p : nullptr;
}

Result<HipLinearInfo> HipPreparedModel::linear_info(std::uint32_t layer, LinearRole role) const {
    const auto* l = find(layer, role);
    if (!l) {
        return Status::invalid_argument(std::string("no resident linear for role ") + to_string(role) + " at layer " +
                                        std::to_string(layer));
    }
    return l->info;
}

Status HipPreparedModel::linear(std::uint32_t layer, LinearRole role, const float* x, float* y, std::uint32_t rows,
                                QuantizedLinearExecutionKind tactic) const {
    const auto* l = find(layer, role);
    if (!l) {
        return Status::invalid_argument(std::string("no resident linear for role ") + to_string(role) + " at layer " +
                                        std::to_string(layer));
    }
    int t = AIR_HIP_LINEAR_AUTO;
    switch (tactic) {
    case QuantizedLinearExecutionKind::hip_decode: t = AIR_HIP_LINEAR_DECODE; break;
    case QuantizedLinearExecutionKind::hip_prefill: t = AIR_HIP_LINEAR_PREFILL; break;
    default:
        return Status::unsupported(std::string("HIP backend does not provide linear tactic ") + to_string(tactic));
    }
    return hip_status(air_hip_linear(ctx_, l->matrix, x, y, l->bias, rows, t));
}

Status HipPreparedModel::linear_epilogue(std::uint32_t layer, LinearRole role, const float* x, std::uint32_t rows,
                                         float* out, int epilogue, const float* norm_weight, float* norm_out,
                                         double eps, QuantizedLinearExecutionKind tactic) const {
    const auto* l = find(layer, role);
    if (!l) {
        return Status::invalid_argument(std::string("no resident linear for role ") + to_string(role) + " at layer " +
                                        std::to_string(layer));
    }
    int t = AIR_HIP_LINEAR_AUTO;
    switch (tactic) {
    case QuantizedLinearExecutionKind::hip_decode: t = AIR_HIP_LINEAR_DECODE; break;
    case QuantizedLinearExecutionKind::hip_prefill: t = AIR_HIP_LINEAR_PREFILL; break;
    default:
        return Status::unsupported(std::string("HIP backend does not provide linear tactic ") + to_string(tactic));
    }
    return hip_status(
        air_hip_linear_epilogue(ctx_, l->matrix, x, rows, out, l->bias, epilogue, norm_weight, norm_out, eps, t));
}

Status HipPreparedModel::linear_rope_kv(std::uint32_t layer, LinearRole role, const float* x, std::uint32_t rows,
                                        float* qkv, const air_hip_kv_layout* kv, const std::int32_t* positions,
                                        const std::int32_t* page_tables, std::uint32_t q_heads,
                                        std::uint32_t kv_heads, std::uint32_t head_dim, std::uint32_t rope_dims,
                                        const float* rope_table, std::uint64_t table_positions,
                                        QuantizedLinearExecutionKind tactic) const {
    const auto* l = find(layer, role);
    if (!l) {
        return Status::invalid_argument(std::string("no resident linear for role ") + to_string(role) + " at layer " +
                                        std::to_string(layer));
    }
    int t = AIR_HIP_LINEAR_AUTO;
    switch (tactic) {
    case QuantizedLinearExecutionKind::hip_decode: t = AIR_HIP_LINEAR_DECODE; break;
    case QuantizedLinearExecutionKind::hip_prefill: t = AIR_HIP_LINEAR_PREFILL; break;
    default:
        return Status::unsupported(std::string("HIP backend does not provide linear tactic ") + to_string(tactic));
    }
    return hip_status(air_hip_linear_rope_kv(ctx_, l->matrix, x, rows, qkv, l->bias, kv, positions, page_tables, layer,
                                             q_heads, kv_heads, head_dim, rope_dims, rope_table, table_positions, t));
}

Status HipPreparedModel::decode_linear_fused(std::uint32_t layer, LinearRole role, const float* x, float* y,
                                             const float* norm_weight, double eps, int epilogue) const {
    const auto* l = find(layer, role);
    if (!l) {
        return Status::invalid_argument(std::string("no resident linear for role ") + to_string(role) + " at layer " +
                                        std::to_string(layer));
    }
    return hip_status(air_hip_decode_linear_fused(ctx_, l->matrix, x, y, l->bias, norm_weight, eps, epilogue));
}

Status HipPreparedModel::set_stream(void* stream) {
    if (Status s = hip_status(air_hip_context_set_stream(ctx_, stream)); !s) return s;
    options_.stream = stream;
    return Status::ok();
}

Status HipPreparedModel::synchronize() const {
    if (Status s = runtime_status(hipSetDevice(device_), "hipSetDevice"); !s) return s;
    return runtime_status(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

Result<HipStepEngine*> HipPreparedModel::engine_for(const ExecutionPlan& plan) {
    const std::uint32_t page_tokens = plan.kv.page_tokens.value_or(0U);
    if (page_tokens == 0U) return Status::invalid_argument("HIP sequences need a KV page size");
    if (page_tokens != options_.kv_page_tokens) {
        // Capacity and admission are answered in the prepared page size.
        return Status::invalid_argument("HIP model is prepared for " + std::to_string(options_.kv_page_tokens) +
                                        "-token KV pages, plan asks for " + std::to_string(page_tokens));
    }
    if (engine_) {
        if (engine_->page_tokens() != page_tokens) {
            return Status::invalid_argument("HIP KV pool already uses " + std::to_string(engine_->page_tokens()) +
                                            "-token pages");
        }
        return engine_.get();
    }
    auto engine = HipStepEngine::create(*this, page_tokens, options_.kv_pool_pages, options_.max_step_rows);
    if (!engine) return engine.status();
    engine_ = std::move(engine).value();
    return engine_.get();
}

Result<std::unique_ptr<runtime_detail::SequenceState>> HipPreparedModel::create_sequence(const ExecutionPlan& plan) {
    if (Status s = validate_execution_plan(plan, capabilities_); !s) return s;
    auto engine = engine_for(plan);
    if (!engine) return engine.status();
    return std::unique_ptr<runtime_detail::SequenceState>(
        std::make_unique<HipSequence>(*engine.value(), plan.linear, plan.attention));
}

std::uint64_t HipPreparedModel::kv_pool_allocated_bytes() const noexcept {
    return engine_ ? engine_->pool_bytes() : 0U;
}

std::uint32_t HipPreparedModel::engine_chunk_pages() const noexcept {
    return engine_ ? engine_->chunk_pages() : 0U;
}

std::uint64_t HipPreparedModel::kv_pool_free_bytes() const noexcept {
    return engine_ ? engine_->free_pool_bytes() : 0U;
}

// Rows of every item packed into device steps of up to max_step_rows rows (a
// sequence's prompt may span steps; its rows stay in order).  A step runs one
// tactic pair, so a change of tactics between items starts a new step.
Result<runtime_detail::PrefillBatchExecution> HipPreparedModel::prefill_batch(
    std::span<const runtime_detail::PrefillBatchItem> items) {
    runtime_detail::PrefillBatchExecution execution;
    execution.items.resize(items.size());
    if (items.empty()) return execution;
    if (!engine_) return Status::invalid_state("no HIP sequence has been created");
    for (const auto& item : items) {
        if (!dynamic_cast<HipSequence*>(item.sequence)) return Status::invalid_argument("prefill item is not a HIP sequence");
        if (item.tokens.empty()) return Status::invalid_argument("prefill requires at least one token");
    }
    HipStepEngine* engine = engine_.get();
    std::vector<StepRow> rows;
    std::vector<std::size_t> owner;  // item of each row with an output
    QuantizedLinearExecutionKind block = QuantizedLinearExecutionKind::hip_decode;
    QuantizedLinearExecutionKind output = QuantizedLinearExecutionKind::hip_decode;
    AttentionExecutionKind attention = AttentionExecutionKind::baseline;
    const auto flush = [&]() -> Status {
        if (rows.empty()) return Status::ok();
        auto result = engine->run(rows, block, output, attention);
        if (!result) return result.status();
        std::size_t g = 0, l = 0, o = 0;
        for (const auto& row : rows) {
            if (row.output == RowOutput::none) continue;
            auto& item = execution.items[owner[o++]];
            if (row.output == RowOutput::greedy) item.greedy_token = result.value().greedy[g++];
            if (row.output == RowOutput::logits) item.logits = std::move(result.value().logits[l++]);
        }
        ++execution.physical_batches;
        execution.physical_tokens += rows.size();
        rows.clear();
        owner.clear();
        return Status::ok();
    };
    std::uint32_t sequences = 0;
    for (std::size_t i = 0; i < items.size(); ++i) {
        auto* seq = static_cast<HipSequence*>(items[i].sequence);
        if (!rows.empty() && (seq->prefill_block_tactic() != block || seq->decode_output_tactic() != output ||
                              seq->prefill_attention() != attention)) {
            if (Status s = flush(); !s) return s;
        }
        block = seq->prefill_block_tactic();
        output = seq->decode_output_tactic();
        attention = seq->prefill_attention();
        ++sequences;
        for (std::size_t t = 0; t < items[i].tokens.size(); ++t) {
            StepRow row{seq, items[i].tokens[t], RowOutput::none};
            if (t + 1 == items[i].tokens.size()) {
                row.output = items[i].output == runtime_detail::PrefillBatchOutput::greedy   ? RowOutput::greedy
                             : items[i].output == runtime_detail::PrefillBatchOutput::logits ? RowOutput::logits
                                                                                             : RowOutput::none;
                if (row.output != RowOutput::none) owner.push_back(i);
            }
            rows.push_back(row);
            if (rows.size() == engine->max_rows()) {
                if (Status s = flush(); !s) return s;
            }
        }
        ++execution.physical_sequence_participations;
    }
    if (Status s = flush(); !s) return s;
    execution.max_sequences = sequences;
    return execution;
}

Result<StepResult> HipPreparedModel::decode_rows(std::span<const runtime_detail::GreedyDecodeBatchItem> items,
                                                 RowOutput output) {
    if (!engine_) return Status::invalid_state("no HIP sequence has been created");
    if (items.size() > capabilities_.max_decode_batch_width) {
        return Status::invalid_argument("decode batch exceeds the advertised width");
    }
    // One launch runs one tactic set: the first item's; items whose plan
    // differs are refused (the service batches only matching plans).
    std::vector<StepRow> rows;
    const HipSequence* first = nullptr;
    for (const auto& item : items) {
        auto* seq = dynamic_cast<HipSequence*>(item.sequence);
        if (!seq) return Status::invalid_argument("decode item is not a HIP sequence");
        for (const auto& row : rows) {
            if (row.sequence == seq) return Status::invalid_argument("a sequence appears twice in a decode batch");
        }
        if (!first) first = seq;
        if (seq->decode_block_tactic() != first->decode_block_tactic() ||
            seq->decode_output_tactic() != first->decode_output_tactic() ||
            seq->decode_attention() != first->decode_attention()) {
            return Status::invalid_argument("decode batch mixes execution plans");
        }
        rows.push_back({seq, item.token, output});
    }
    return engine_->run(rows, first->decode_block_tactic(), first->decode_output_tactic(), first->decode_attention());
}

Result<std::vector<TokenId>> HipPreparedModel::decode_greedy_batch(
    std::span<const runtime_detail::GreedyDecodeBatchItem> items) {
    if (items.empty()) return std::vector<TokenId>{};
    auto result = decode_rows(items, RowOutput::greedy);
    if (!result) return result.status();
    return std::move(result.value().greedy);
}

Result<std::vector<std::vector<float>>> HipPreparedModel::decode_batch_logits(
    std::span<const runtime_detail::GreedyDecodeBatchItem> items) {
    if (items.empty()) return std::vector<std::vector<float>>{};
    auto result = decode_rows(items, RowOutput::logits);
    if (!result) return result.status();
    return std::move(result.value().logits);
}

Result<std::unique_ptr<runtime_detail::SequenceState>> HipPreparedModel::restore_sequence(
    const ExecutionPlan& plan, const runtime_detail::SequenceCheckpoint& checkpoint) {
    if (Status s = validate_execution_plan(plan, capabilities_); !s) return s;
    if (checkpoint.backend() != BackendKind::hip) {
        return Status::invalid_argument("HIP backend cannot restore a checkpoint from another backend");
    }
    return Status::unsupported("HIP sequences do not provide checkpoints");
}

std::uint64_t HipPreparedModel::resident_device_bytes() const noexcept {
    air_hip_stats stats{};
    if (air_hip_context_stats(ctx_, &stats) != AIR_HIP_OK) return bias_bytes_;
    return stats.resident_matrix_bytes + stats.workspace_bytes + bias_bytes_ +
           (engine_ ? engine_->resident_bytes() : 0U);
}

std::uint64_t HipPreparedModel::estimate_sequence_device_bytes(const ExecutionPlan& plan,
                                                               std::uint64_t max_tokens) const noexcept {
    return estimate_paged_fp32_sequence_bytes(model_->config(), plan.kv.page_tokens.value_or(0U), max_tokens);
}

std::uint64_t estimate_paged_fp32_sequence_bytes(const ModelConfig& c, std::uint32_t page_tokens,
                                                 std::uint64_t max_tokens) noexcept {
    constexpr auto kMax = std::numeric_limits<std::uint64_t>::max();
    if (page_tokens == 0U || max_tokens == 0U || c.attention_head_count == 0U) return 0U;
    const std::uint64_t head = c.embedding_size / c.attention_head_count;
    const std::uint64_t kv_width = static_cast<std::uint64_t>(c.kv_head_count) * head;
    const std::uint64_t bytes_per_token = static_cast<std::uint64_t>(c.layer_count) * kv_width * 2U * sizeof(float);
    if (bytes_per_token == 0U) return 0U;
    const std::uint64_t pages = (max_tokens + page_tokens - 1U) / page_tokens;
    if (pages > kMax / (static_cast<std::uint64_t>(page_tokens) * bytes_per_token)) return kMax;
    const std::uint64_t page_bytes = static_cast<std::uint64_t>(page_tokens) * bytes_per_token;
    const std::uint64_t max_pages = (c.context_length + page_tokens - 1U) / page_tokens;
    if (max_pages > kMax / (2U * sizeof(float*))) return kMax;
    const std::uint64_t table_bytes = max_pages * 2U * sizeof(float*);
    const std::uint64_t kv_bytes = pages * page_bytes;
    if (kv_bytes > kMax - table_bytes) return kMax;
    return kv_bytes + table_bytes;
}

std::optional<std::uint64_t> HipPreparedModel::free_device_bytes() const {
    std::uint64_t free = 0, total = 0;
    if (air_hip_mem_info(device_, &free, &total) != AIR_HIP_OK) return std::nullopt;
    return free;
}

// A growing pool (the default): the device memory free now plus the pool
// already allocated, the reference's answer (src/runtime/backend.cpp:541-560);
// unknown when the free memory cannot be read.  A fixed pool: that pool (before
// the first sequence, the pool it will allocate), since it never grows.
std::optional<std::uint64_t> HipPreparedModel::sequence_capacity_bytes() const {
    if (options_.kv_pool_pages) {
        if (engine_) return engine_->pool_bytes();
        return static_cast<std::uint64_t>(HipStepEngine::planned_pool_pages(*this, options_.kv_page_tokens)) *
               HipStepEngine::kv_page_bytes(model_->config(), options_.kv_page_tokens);
    }
    const auto free = free_device_bytes();
    if (!free) return std::nullopt;
    const std::uint64_t pool = kv_pool_allocated_bytes();
    if (*free > std::numeric_limits<std::uint64_t>::max() - pool) return std::numeric_limits<std::uint64_t>::max();
    return *free + pool;
}

Result<std::unique_ptr<runtime_detail::PreparedModel>> prepare_hip_model(std::shared_ptr<const ModelDefinition> model,
                                                                         int device_ordinal) {
    HipPrepareOptions options;
    options.device = device_ordinal;
    auto prepared = HipPreparedModel::create(std::move(model), options);
    if (!prepared) return prepared.status();
    return std::unique_ptr<runtime_detail::PreparedModel>(std::move(prepared).value());
}

} // namespace air

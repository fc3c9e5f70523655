// Engine configuration (include/zcgvs/engine/engine_config.hpp). Every field of the reference is
// kept so existing configurations load unchanged. Fields that name components outside this
// build's scope (tokenizer vocabulary, ONNX encoder and reranker models) are accepted and
// recorded; text queries then need a QueryEmbedder attached at run time.
#pragma once

#include <string>

#include "zcgvs/core/metric.hpp"
#include "zcgvs/search/search_params.hpp"

namespace zcgvs {

enum class RerankerBackend { Onnx };

struct EngineConfig {
    std::string embeddings_path;
    std::string metadata_path;  // empty: ids are the corpus indices, passages are empty
    std::string vocab_path;
    std::string rescore_embeddings_path;
    std::string lexical_index_path;
    std::string encoder_model_path;
    std::string encoder_output_name = "last_hidden_state";
    int encoder_max_seq_len = 256;
    RerankerBackend reranker_backend = RerankerBackend::Onnx;
    std::string reranker_model_path;
    std::string reranker_output_name = "logits";
    int reranker_max_seq_len = 256;
    int reranker_batch_size = 32;
    int device_id = 0;
    bool lowercase = true;
    Metric metric = Metric::Cosine;
    SimilarityBackend similarity_backend = SimilarityBackend::Custom;
    int default_top_k = 10;
    int default_candidates = 100;
    int rescore_candidates = 0;  // 0 disables rescoring even with a rescore store
    bool hybrid = false;         // run the BM25 stage by default when an index is attached
    float dense_weight = 0.7f;
    int max_query_terms = 64;
    bool use_cuda_graphs = false;  // replay the device pipeline from an instantiated HIP graph
};

}  // namespace zcgvs

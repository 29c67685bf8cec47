// Tokenizers: the reference's encode layers (kuiper/include/op/encode.h:17-89),
// CPU text I/O in front of the decode loop, with the same classes and
// methods.  Everything is self-contained C++ (no sentencepiece, RE2, abseil or
// JSON library):
//
//  * SpeEncodeLayer reads a SentencePiece model file (the protobuf
//    ModelProto) and encodes with its BPE algorithm: whitespace escaped as
//    U+2581 after a dummy prefix, symbols merged highest piece score first,
//    pieces outside the vocabulary as <0xXX> byte pieces (byte fallback) or
//    the unknown id.  Models of another type or with a non-identity
//    normaliser are refused (init() reports it).
//  * BpeEncodeLayer / QwenEncodeLayer read a HF tokenizer.json ("model" ->
//    "vocab" and "added_tokens") and encode as the reference's tiktoken path:
//    the byte-level vocabulary mapped back to raw bytes, a token's id is its
//    merge rank, special tokens matched anywhere, the text between them split
//    by the reference's pre-tokenizer pattern (encode.cpp:61-62, matched here
//    by hand), each piece looked up whole or byte-pair merged lowest rank
//    first.  As in the reference, encode() replaces every " " with U+0120
//    first and decode() maps U+0120 back to " ".
//
// A layer that could not load its file reports it from init(); its encode()
// then returns no ids and decode() an empty string.  Where the reference
// aborts or throws on bad input, these layers do not: decode() skips ids it
// does not know, a tokenizer.json whose vocabulary lacks one of the 256 byte
// tokens is refused at init(), and a special token the layer names (BOS, EOS,
// second stop token) that the file does not hold gets id -1, where the
// reference's map lookup would add it with id 0.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "kuiper/layer.h"

namespace op {

class EncodeLayerBase : public Layer {
 public:
  explicit EncodeLayerBase(std::string token_model_path, bool has_bos, bool has_eos)
      : Layer(base::DeviceType::kDeviceCPU, LayerType::kLayerEncode, "Encode"),
        has_bos_(has_bos),
        has_eos_(has_eos),
        token_model_path_(std::move(token_model_path)) {}

  virtual std::vector<int32_t> encode(const std::string& sentence) const = 0;
  virtual std::string decode(int32_t token_id) const = 0;
  virtual std::string decode(const std::vector<int32_t>& token_ids) const = 0;
  virtual bool is_sentence_ending(int32_t token_id) const = 0;
  virtual int32_t vocab_size() const = 0;

  // Whether the tokenizer file was read (the reference aborts instead).
  base::Status init() override { return status_; }

 protected:
  bool has_bos_ = true;
  bool has_eos_ = false;
  std::string token_model_path_;
  base::Status status_;
};

// SentencePiece BPE model (kuiper/source/op/encode.cpp:14-57).
class SpeEncodeLayer : public EncodeLayerBase {
 public:
  explicit SpeEncodeLayer(std::string token_model_path, bool has_bos, bool has_eos);
  std::vector<int32_t> encode(const std::string& sentence) const override;
  std::string decode(int32_t token_id) const override;
  std::string decode(const std::vector<int32_t>& token_ids) const override;
  bool is_sentence_ending(int32_t token_id) const override;
  int32_t vocab_size() const override;

  int32_t bos_id() const { return bos_id_; }
  int32_t eos_id() const { return eos_id_; }

 private:
  struct Piece {
    std::string text;
    float score = 0.f;
    int type = 1;  // 1 normal, 2 unknown, 3 control, 4 user defined, 5 unused, 6 byte
  };
  std::vector<Piece> pieces_;
  std::unordered_map<std::string, int32_t> index_;  // normal / user-defined pieces
  int32_t byte_ids_[256];
  int32_t unk_id_ = 0, bos_id_ = 1, eos_id_ = 2;
  bool byte_fallback_ = false;
  bool add_dummy_prefix_ = true;
  bool remove_extra_whitespaces_ = false;
  bool escape_whitespaces_ = true;
};

// Byte-level BPE from a tokenizer.json, Llama-3 special tokens
// (kuiper/source/op/encode.cpp:64-146).
class BpeEncodeLayer : public EncodeLayerBase {
 public:
  explicit BpeEncodeLayer(std::string token_model_path, bool has_bos, bool has_eos);
  std::vector<int32_t> encode(const std::string& sentence) const override;
  std::string decode(int32_t token_id) const override;
  std::string decode(const std::vector<int32_t>& token_ids) const override;
  bool is_sentence_ending(int32_t token_id) const override;
  int32_t vocab_size() const override;

  int32_t bos_id() const { return bos_id_; }
  int32_t eos_id() const { return eos_id_; }

 protected:
  struct Deferred {};
  // For subclasses that load() with their own special-token names.
  BpeEncodeLayer(Deferred, std::string token_model_path, bool has_bos, bool has_eos);
  // Reads the file; names the BOS, EOS and second stop token.
  void load(const char* bos, const char* eos, const char* stop2);
  std::vector<int32_t> encode_ordinary(const std::string& text) const;
  void byte_pair_merge(const std::string& piece, std::vector<int32_t>& out) const;

  int32_t bos_id_ = -1;
  int32_t eos_id_ = -1;
  int32_t stop_token1_ = -1;
  int32_t stop_token2_ = -1;
  int32_t num_token_ = 0;
  std::unordered_map<std::string, int32_t> encoder_;       // raw bytes -> rank (= id)
  std::unordered_map<int32_t, std::string> decoder_;
  std::vector<std::pair<std::string, int32_t>> special_;   // special tokens, longest first
  std::unordered_map<int32_t, std::string> special_decoder_;
};

// The same with the Qwen special tokens (kuiper/source/op/encode.cpp:148-182).
class QwenEncodeLayer : public BpeEncodeLayer {
 public:
  explicit QwenEncodeLayer(std::string token_model_path, bool has_bos, bool has_eos);
};

}  // namespace op

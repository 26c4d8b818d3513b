// Byte-level BPE of a Hugging Face tokenizer.json, host side: the tokenizer behind
// accel_llama_tokenizer / encode / decode / complete (AccelEP's accel::Bpe,
// include/accel/bpe.h, src/bpe.cc). Plain C++ with no HIP dependency; errors are thrown as
// std::invalid_argument with a message.
//
// The accepted files are the SmolLM2 form: model BPE (vocab, merges), no normalizer and no
// post-processor, a pre-tokenizer sequence of Digits (individual digits) then ByteLevel
// (no prefix space, regex on), a ByteLevel decoder, and added tokens in the vocabulary.
#pragma once

#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace accel_hip {

class ByteBpe {
 public:
  ByteBpe();

  // Reads and checks a tokenizer.json; on failure the tokenizer is left unloaded.
  void Load(const std::string& path);
  bool loaded() const { return loaded_; }
  int32_t vocab_size() const { return static_cast<int32_t>(tokens_.size()); }

  // Token ids of `text` (UTF-8 bytes, NUL allowed): added tokens are matched first (the
  // longest at each position, the earliest listed on a tie), the text between them goes
  // through the digit split, the GPT-2 pattern, the byte mapping and the merges.
  std::vector<int32_t> Encode(std::string_view text) const;
  // UTF-8 text of the ids; skip_special leaves out tokens marked special. Byte sequences
  // that are not valid UTF-8 come out as U+FFFD, one per offending byte.
  std::string Decode(const int32_t* ids, int32_t count, bool skip_special) const;

 private:
  void EncodeSegment(std::string_view segment, std::vector<int32_t>& out) const;
  void EncodeWord(const std::vector<int32_t>& symbols, std::vector<int32_t>& out) const;
  size_t LongestAdded(std::string_view text, size_t pos, int32_t* id) const;

  struct AddedToken {
    std::string text;
    int32_t id;
  };
  struct MergeRule {
    uint32_t rank;
    int32_t result;
  };

  bool loaded_ = false;
  std::vector<std::string> tokens_;    // id -> token text (byte-level alphabet for BPE tokens)
  std::vector<uint8_t> special_;       // id -> marked special in added_tokens
  std::vector<AddedToken> added_;      // in file order
  std::unordered_map<uint64_t, MergeRule> merges_;  // (left id << 32 | right id) -> rule
  int32_t byte_token_[256];            // id of the one-byte token of each byte, or -1
  // The byte-level alphabet: byte b is written as code point alphabet_[b]; reverse_ maps a
  // code point back to its byte.
  char32_t alphabet_[256];
  std::unordered_map<char32_t, uint8_t> reverse_;
};

}  // namespace accel_hip

// gn_tools.h - host-side pieces of the rollout state machine: gonano's
// byte-level tokenizer ids and the calculator tool.
#pragma once

#include <optional>
#include <string>
#include <vector>

namespace gn {

// tokenizer/special.go:19-31 appended after the 256 byte ranks.
enum SpecialToken : int {
  TOK_BOS = 256,
  TOK_USER_START = 257,
  TOK_USER_END = 258,
  TOK_ASSISTANT_START = 259,
  TOK_ASSISTANT_END = 260,
  TOK_TOOL_START = 261,
  TOK_TOOL_END = 262,
  TOK_TOOL_OUTPUT_START = 263,
  TOK_TOOL_OUTPUT_END = 264,
  TOK_THINK_START = 265,
  TOK_THINK_END = 266,
  TOKENIZER_VOCAB = 267,
};

// Tokenizer.Decode (tokenizer/tokenizer.go:110-118): bytes for ids < 256,
// special names for 256..266, other ids skipped.
std::string decode_tokens(const std::vector<int>& ids);
// Tokenizer.Encode for the byte-level tokenizer: one id per byte.
std::vector<int> encode_bytes(const std::string& s);
// Calculator.Call (inference/tooluse.go:27-47).
std::optional<std::string> calculator(const std::string& expr);

}  // namespace gn

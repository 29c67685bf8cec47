// kuiper_generate: the generate/serve driver of the reference demos
// (demo/main.cpp:5-47, demo/main_qwen.cpp:198-284 and :404-452) on the
// MI355X backend, through the C++ host API (model::Model on kDeviceHIP).
//
// Without a tokenizer, prompts and responses are token ids:
//
//   kuiper_generate [options] <model.bin> <ids> [max_new_tokens]
//       ids: comma- or space-separated prompt token ids.  Prints
//       [RESPONSE_START] / generated ids / [RESPONSE_END] on stdout and
//       [STATS] steps=.. duration=.. steps_per_s=.. on stderr.
//   kuiper_generate --serve [options] <model.bin> [max_new_tokens]
//       prints [READY]; then for each block of lines between [PROMPT_START]
//       and [PROMPT_END] (token ids) prints one response as above; [EXIT] or
//       end of input stops.
//
// With --tokenizer FILE (a SentencePiece .model for llama2, a tokenizer.json
// for the other families) the prompt is text, as in the reference demos: the
// single-shot <ids> argument becomes <prompt>, a served prompt is its lines
// joined by "\n", and the response is decoded text with the end markers cut
// and short repeated lines collapsed (main_qwen.cpp:94-148).  The prompt and
// response ids then go to stderr as [PROMPT_IDS] / [RESPONSE_IDS] lines.
//
// Options: --family llama2|llama3|qwen2|qwen3 (default llama2), --quant (int8
// image), --layered (the layer-by-layer path instead of the fused engine),
// --prefill (the whole prompt in one batched pass; fused only), --eos ID
// (end-of-sequence id, repeatable), --tokenizer FILE, --profile (per-operation
// device times of the generation on stderr, one [PROFILE] line per operation:
// the reference's op profile, main_qwen.cpp:287-310, timed on the device).
//
// Generation follows main_qwen.cpp: prompt positions advance without
// sampling; in the decode phase only, generation stops at an end-of-sequence
// id (the tokenizer's and --eos ones), after 24 identical tokens in a row,
// when the last 12 tokens repeat the 12 before them, or, with a tokenizer,
// when the decoded last 6 tokens hold an end marker.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "kuiper/model.h"

namespace {

struct Options {
  model::ModelFamily family = model::ModelFamily::kLlama2;
  bool quant = false;
  bool layered = false;
  bool prefill = false;
  std::vector<int32_t> eos;
  std::string tokenizer;
  bool profile = false;
};

struct GenerationResult {
  std::vector<int32_t> response;
  int32_t steps = 0;
};

std::vector<int32_t> parse_ids(const std::string& text, bool* ok) {
  std::vector<int32_t> ids;
  std::string t = text;
  for (char& c : t)
    if (c == ',') c = ' ';
  std::istringstream in(t);
  std::string w;
  *ok = true;
  while (in >> w) {
    char* end = nullptr;
    const long v = std::strtol(w.c_str(), &end, 10);
    if (*end != '\0' || v < 0 || v > 0x7fffffffL) {
      *ok = false;
      return {};
    }
    ids.push_back(static_cast<int32_t>(v));
  }
  return ids;
}

const char* const kEndMarkers[] = {"<|im_end|>", "<|endoftext|>", "</s>", "<|end|>"};

bool has_end_marker(const std::string& text) {
  for (const char* mk : kEndMarkers)
    if (text.find(mk) != std::string::npos) return true;
  return false;
}

std::string trim(const std::string& text) {
  const size_t b = text.find_first_not_of(" \t\r\n");
  if (b == std::string::npos) return "";
  const size_t e = text.find_last_not_of(" \t\r\n");
  return text.substr(b, e - b + 1);
}

// main_qwen.cpp:94-148: the text before the first end marker (each marker in
// turn), then runs of one short line cut: the second repeat of a line of at
// most 32 characters ends the text and drops the first repeat; lines of up to
// 48 characters are kept at most twice in a row.
std::string response_text(const std::string& decoded) {
  std::string text = decoded;
  for (const char* mk : kEndMarkers) {
    const size_t at = text.find(mk);
    if (at != std::string::npos) text = text.substr(0, at);
  }
  text = trim(text);
  std::istringstream in(text);
  std::string line, prev;
  std::vector<std::string> kept;
  int run = 0;
  while (std::getline(in, line)) {
    const std::string norm = trim(line);
    if (!norm.empty() && norm == prev && norm.size() <= 48) {
      ++run;
      if (run >= 2 && norm.size() <= 32) {
        if (!kept.empty() && trim(kept.back()) == norm) kept.pop_back();
        break;
      }
      if (run >= 3) continue;
    } else {
      prev = norm;
      run = 1;
    }
    kept.push_back(line);
  }
  std::string out;
  for (size_t i = 0; i < kept.size(); ++i) out += (i ? "\n" : "") + kept[i];
  return trim(out);
}

void print_profile(const model::Model& m) {
  for (const model::OpProfileStat& st : m.get_profile_stats())
    std::fprintf(stderr, "[PROFILE] op=%s calls=%lld total_ms=%.4f avg_ms=%.5f\n", st.op_name.c_str(),
                 static_cast<long long>(st.calls), st.total_ms, st.avg_ms);
  std::fflush(stderr);
}

std::string join_ids(const std::vector<int32_t>& ids) {
  std::string out;
  for (size_t i = 0; i < ids.size(); ++i) out += (i ? " " : "") + std::to_string(ids[i]);
  return out;
}

// main_qwen.cpp:198-284 with token ids.
// Why a prompt cannot run on the model ("" when it can): ids outside
// [0, vocab) or more positions than the model's sequence length.
std::string prompt_error(const model::Model& m, const std::vector<int32_t>& prompt) {
  const auto& c = m.config();
  for (int32_t t : prompt) {
    if (t < 0 || t >= c.vocab_size_)
      return "token id " + std::to_string(t) + " is outside [0, " + std::to_string(c.vocab_size_) +
             ")";
  }
  if (static_cast<int64_t>(prompt.size()) > c.seq_len_)
    return "the prompt has " + std::to_string(prompt.size()) + " tokens; the model holds " +
           std::to_string(c.seq_len_) + " positions";
  return "";
}

GenerationResult generate(const model::Model& m, const std::vector<int32_t>& prompt, int max_new,
                          bool use_prefill, bool has_tokenizer) {
  GenerationResult r;
  const int32_t P = static_cast<int32_t>(prompt.size());
  const int32_t total_steps =
      std::min<int32_t>(P + std::max(1, max_new), m.config().seq_len_);
  tensor::Tensor pos_tensor = m.get_buffer(model::ModelBufferType::kInputPos);
  std::vector<int32_t> words(prompt.begin(), prompt.begin() + 1);
  int32_t pos = 0, next = prompt[0], last = -1, same_run = 0;
  bool is_prompt = true;
  if (use_prefill && P >= 2) {
    // The prompt in one batched pass: the loop resumes at the first sampled
    // token, as if positions 0 .. P-1 had run one by one.
    int nx = -1;
    STATUS_CHECK(m.prefill(prompt, nx));
    words.assign(prompt.begin(), prompt.end());
    next = nx;
    pos = P;
    is_prompt = false;
    if (!m.is_sentence_ending(next)) {
      words.push_back(next);
      r.response.push_back(next);
      last = next;
      same_run = 1;
    } else {
      r.steps = pos;
      return r;
    }
  } else {
    const op::EmbeddingOutput prompt_embedding = m.embedding(prompt);
    while (pos < total_steps && pos < P - 1) {
      pos_tensor.index<int32_t>(0) = pos;
      STATUS_CHECK(m.predict(m.fill_input(pos_tensor, prompt_embedding, true), pos_tensor, true,
                             next));
      next = prompt[pos + 1];
      words.push_back(next);
      ++pos;
    }
  }
  while (pos < total_steps) {
    pos_tensor.index<int32_t>(0) = pos;
    is_prompt = false;
    const op::EmbeddingOutput emb = m.embedding({next});
    STATUS_CHECK(m.predict(m.fill_input(pos_tensor, emb, false), pos_tensor, false, next));
    if (m.is_sentence_ending(next)) break;
    words.push_back(next);
    r.response.push_back(next);
    // 1) the same token 24 times in a row
    if (next == last) {
      ++same_run;
    } else {
      last = next;
      same_run = 1;
    }
    if (same_run >= 24) break;
    // 2) an end marker in the decoded last 6 tokens (with a tokenizer)
    if (has_tokenizer && words.size() > static_cast<size_t>(P + 6)) {
      const std::string tail = m.decode(std::vector<int32_t>(words.end() - 6, words.end()));
      if (has_end_marker(tail)) break;
    }
    // 3) the last 12 tokens repeat the 12 before them
    constexpr int kRepeatWindow = 12;
    if (words.size() >= static_cast<size_t>(P + kRepeatWindow * 2)) {
      bool repeated = true;
      auto e = words.end();
      for (int i = 0; i < kRepeatWindow && repeated; ++i)
        repeated = *(e - 1 - i) == *(e - 1 - kRepeatWindow - i);
      if (repeated) break;
    }
    ++pos;
  }
  (void)is_prompt;
  r.steps = pos;
  return r;
}

// main_qwen.cpp:378-387.  With a tokenizer the response is text and the ids
// go to stderr.
void print_result(const model::Model& m, const GenerationResult& r, double duration_sec,
                  bool print_stats, bool has_tokenizer) {
  const double sps = duration_sec > 0 ? static_cast<double>(r.steps) / duration_sec : 0.0;
  if (has_tokenizer) {
    const std::string text = r.response.empty() ? "" : response_text(m.decode(r.response));
    std::printf("[RESPONSE_START]\n%s\n[RESPONSE_END]\n", text.c_str());
    std::fprintf(stderr, "[RESPONSE_IDS] %s\n", join_ids(r.response).c_str());
    std::fflush(stderr);
  } else {
    std::printf("[RESPONSE_START]\n%s\n[RESPONSE_END]\n", join_ids(r.response).c_str());
  }
  std::fflush(stdout);
  if (print_stats) {
    std::fprintf(stderr, "[STATS] steps=%d duration=%.6f steps_per_s=%.6f\n", r.steps,
                 duration_sec, sps);
    std::fflush(stderr);
  }
}

std::unique_ptr<model::Model> load(const std::string& path, const Options& o) {
  std::unique_ptr<model::Model> m;
  switch (o.family) {
    case model::ModelFamily::kQwen2:
      m = std::make_unique<model::Qwen2Model>(base::TokenizerType::kEncodeBpe, o.tokenizer, path,
                                              o.quant);
      break;
    case model::ModelFamily::kQwen3:
      m = std::make_unique<model::Qwen3Model>(base::TokenizerType::kEncodeBpe, o.tokenizer, path,
                                              o.quant);
      break;
    case model::ModelFamily::kLlama3:
      m = std::make_unique<model::LLama2Model>(base::TokenizerType::kEncodeBpe, o.tokenizer, path,
                                               o.quant, o.family);
      break;
    default:
      m = std::make_unique<model::LLama2Model>(base::TokenizerType::kEncodeSpe, o.tokenizer, path,
                                               o.quant, o.family);
  }
  const base::Status s = m->init(base::DeviceType::kDeviceHIP);
  if (!s) {
    std::fprintf(stderr, "kuiper_generate: init failed (%d): %s\n", int(s), s.get_err_msg().c_str());
    return nullptr;
  }
  if (!o.layered) STATUS_CHECK(m->set_fused(true));
  m->set_eos_tokens(o.eos);
  return m;
}

int usage(const char* prog) {
  std::fprintf(stderr,
               "Usage:\n  %s [options] <model.bin> <ids|prompt> [max_new_tokens]\n"
               "  %s --serve [options] <model.bin> [max_new_tokens]\n"
               "Options: --family llama2|llama3|qwen2|qwen3, --quant, --layered, --prefill, "
               "--eos ID, --tokenizer FILE (prompts and responses as text), --profile\n",
               prog, prog);
  return 2;
}

int parse_max(const char* s) {
  const int v = std::atoi(s);
  return v > 0 ? v : 128;
}

}  // namespace

int main(int argc, char** argv) {
  Options o;
  bool serve = false;
  std::vector<std::string> pos_args;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--serve") {
      serve = true;
    } else if (a == "--quant") {
      o.quant = true;
    } else if (a == "--layered") {
      o.layered = true;
    } else if (a == "--prefill") {
      o.prefill = true;
    } else if (a == "--eos" && i + 1 < argc) {
      o.eos.push_back(std::atoi(argv[++i]));
    } else if (a == "--profile") {
      o.profile = true;
    } else if (a == "--tokenizer" && i + 1 < argc) {
      o.tokenizer = argv[++i];
      if (o.tokenizer.empty()) return usage(argv[0]);
    } else if (a == "--family" && i + 1 < argc) {
      const std::string f = argv[++i];
      if (f == "llama2") o.family = model::ModelFamily::kLlama2;
      else if (f == "llama3") o.family = model::ModelFamily::kLlama3;
      else if (f == "qwen2") o.family = model::ModelFamily::kQwen2;
      else if (f == "qwen3") o.family = model::ModelFamily::kQwen3;
      else return usage(argv[0]);
    } else if (a.size() > 2 && a[0] == '-' && a[1] == '-') {
      return usage(argv[0]);
    } else {
      pos_args.push_back(a);
    }
  }
  if (o.prefill && o.layered) {
    std::fprintf(stderr, "kuiper_generate: --prefill runs on the fused engine, not --layered\n");
    return 2;
  }
  if (serve) {
    if (pos_args.empty() || pos_args.size() > 2) return usage(argv[0]);
    const int max_steps = pos_args.size() == 2 ? parse_max(pos_args[1].c_str()) : 128;
    auto m = load(pos_args[0], o);
    if (!m) return 1;
    if (o.prefill) STATUS_CHECK(m->set_prefill(true));
    const bool tok = !o.tokenizer.empty();
    std::cout << "[READY]" << std::endl;
    std::string line;
    while (std::getline(std::cin, line)) {
      if (line == "[EXIT]") break;
      if (line != "[PROMPT_START]") continue;
      std::string text;
      bool has_end = false, first = true;
      while (std::getline(std::cin, line)) {
        if (line == "[PROMPT_END]") {
          has_end = true;
          break;
        }
        // Text prompts keep their line breaks (main_qwen.cpp:423-435).
        text += (tok ? (first ? "" : "\n") : " ") + line;
        first = false;
      }
      if (!has_end) break;
      std::vector<int32_t> prompt;
      if (tok) {
        prompt = m->encode(text);
        std::fprintf(stderr, "[PROMPT_IDS] %s\n", join_ids(prompt).c_str());
        if (prompt.empty()) {  // main_qwen.cpp:153-155: an empty response
          print_result(*m, GenerationResult{}, 0.0, false, tok);
          continue;
        }
      } else {
        bool ok = false;
        prompt = parse_ids(text, &ok);
        if (!ok || prompt.empty()) {
          std::printf("[ERROR] the prompt must be token ids\n");
          std::fflush(stdout);
          continue;
        }
      }
      // A bad request gets an error line; it must not reach the model, whose
      // failed checks end the process.
      const std::string why = prompt_error(*m, prompt);
      if (!why.empty()) {
        std::printf("[ERROR] %s\n", why.c_str());
        std::fflush(stdout);
        continue;
      }
      if (o.profile) m->reset_profile_stats();
      const auto t0 = std::chrono::steady_clock::now();
      const GenerationResult r = generate(*m, prompt, max_steps, o.prefill, tok);
      const double dt =
          std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
      print_result(*m, r, dt, false, tok);
      if (o.profile) print_profile(*m);
    }
    return 0;
  }
  if (pos_args.size() < 2 || pos_args.size() > 3) return usage(argv[0]);
  const bool tok = !o.tokenizer.empty();
  std::vector<int32_t> prompt;
  if (!tok) {
    bool ok = false;
    prompt = parse_ids(pos_args[1], &ok);
    if (!ok || prompt.empty()) {
      std::fprintf(stderr, "kuiper_generate: the prompt must be token ids\n");
      return 2;
    }
  }
  const int max_steps = pos_args.size() == 3 ? parse_max(pos_args[2].c_str()) : 128;
  auto m = load(pos_args[0], o);
  if (!m) return 1;
  if (tok) {
    prompt = m->encode(pos_args[1]);
    std::fprintf(stderr, "[PROMPT_IDS] %s\n", join_ids(prompt).c_str());
    if (prompt.empty()) {  // main_qwen.cpp:153-155: an empty response
      print_result(*m, GenerationResult{}, 0.0, true, tok);
      return 0;
    }
  }
  const std::string why = prompt_error(*m, prompt);
  if (!why.empty()) {
    std::fprintf(stderr, "kuiper_generate: %s\n", why.c_str());
    return 2;
  }
  if (o.prefill) STATUS_CHECK(m->set_prefill(true));
  if (o.profile) m->reset_profile_stats();
  const auto t0 = std::chrono::steady_clock::now();
  const GenerationResult r = generate(*m, prompt, max_steps, o.prefill, tok);
  const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  print_result(*m, r, dt, true, tok);
  if (o.profile) print_profile(*m);
  return 0;
}

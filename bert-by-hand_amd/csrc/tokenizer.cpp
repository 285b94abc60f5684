// WordPiece tokenizer of the uncased BERT family: UTF-8 text -> the (batch,
// seq) int32 ids / token types / attention mask that bert_embed takes.
//
// It reproduces the tokenizer the reference calls through
// sentence-transformers (scripts/dump_weights.py:100-106,
// scripts/dump_corpus.py:34-39): Hugging Face tokenizers' BertTokenizerFast
// (tokenizers 0.22.2) with padding="max_length", truncation=True, i.e.
//   normalizer     BertNormalizer: clean text (drop NUL, U+FFFD and other
//                  control characters, map whitespace to ' '), pad CJK
//                  ideographs with spaces, strip accents (NFD, drop
//                  nonspacing marks) when lowercasing, lowercase
//   pre-tokenizer  split on whitespace (dropped) and on punctuation (kept as
//                  one-character words)
//   model          WordPiece: greedy longest match, "##" continuation prefix,
//                  words over 100 characters and unmatchable words -> [UNK]
//   post           [CLS] tokens [SEP], tokens truncated to seq - 2, [PAD] up
//                  to seq; token types 0; mask 1 on real tokens.
// Unicode properties come from unicode_tables.h (generated from Unicode 13.0
// by gen_unicode_tables.py); Hangul syllables are decomposed by formula.

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/bbh.h"
#include "unicode_tables.h"

// Status helpers of the C ABI (capi.hip).
namespace bbh_detail {
bbh_status set_error(bbh_status s, const std::string& msg);
}

struct bbh_tokenizer {
  std::unordered_map<std::string, int32_t> vocab;
  int32_t cls = -1, sep = -1, pad = -1, unk = -1;
  bool lowercase = true;
  int32_t size = 0;
  // special tokens matched verbatim in the raw text before normalisation
  std::vector<std::pair<std::string, int32_t>> specials;
};

namespace {

using bbh_detail::set_error;

int uclass(uint32_t cp) {  // 0 none, 1 other (C*), 2 punctuation (P*), 3 Mn
  int lo = 0, hi = bbh::uni::kClassRanges - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    if (cp < bbh::uni::kClassRange[mid][0])
      hi = mid - 1;
    else if (cp > bbh::uni::kClassRange[mid][1])
      lo = mid + 1;
    else
      return (int)bbh::uni::kClassRange[mid][2];
  }
  return 0;
}

// Unicode White_Space, plus the ASCII controls BERT counts as whitespace.
bool is_whitespace(uint32_t c) {
  return (c >= 0x09 && c <= 0x0D) || c == 0x20 || c == 0x85 || c == 0xA0 || c == 0x1680 ||
         (c >= 0x2000 && c <= 0x200A) || c == 0x2028 || c == 0x2029 || c == 0x202F ||
         c == 0x205F || c == 0x3000;
}

bool is_control(uint32_t c) { return !(c == '\t' || c == '\n' || c == '\r') && uclass(c) == 1; }

bool is_punctuation(uint32_t c) {
  const bool ascii = (c >= 33 && c <= 47) || (c >= 58 && c <= 64) || (c >= 91 && c <= 96) ||
                     (c >= 123 && c <= 126);
  return ascii || uclass(c) == 2;
}

bool is_cjk(uint32_t c) {
  return (c >= 0x4E00 && c <= 0x9FFF) || (c >= 0x3400 && c <= 0x4DBF) ||
         (c >= 0x20000 && c <= 0x2A6DF) || (c >= 0x2A700 && c <= 0x2B73F) ||
         (c >= 0x2B740 && c <= 0x2B81F) || (c >= 0x2B920 && c <= 0x2CEAF) ||
         (c >= 0xF900 && c <= 0xFAFF) || (c >= 0x2F800 && c <= 0x2FA1F);
}

// Binary search of a {cp, offset, length} index.
template <int N>
const uint32_t* find_map(const uint32_t (&index)[N][3], uint32_t cp) {
  int lo = 0, hi = N - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    if (cp < index[mid][0])
      hi = mid - 1;
    else if (cp > index[mid][0])
      lo = mid + 1;
    else
      return index[mid];
  }
  return nullptr;
}

// NFD of one code point with the nonspacing marks dropped.
void push_stripped(uint32_t cp, std::vector<uint32_t>& out) {
  if (cp >= 0xAC00 && cp <= 0xD7A3) {  // Hangul syllable: L V (T) jamo, none of them marks
    const uint32_t s = cp - 0xAC00;
    out.push_back(0x1100 + s / 588);
    out.push_back(0x1161 + (s % 588) / 28);
    if (s % 28) out.push_back(0x11A7 + s % 28);
    return;
  }
  if (const uint32_t* e = find_map(bbh::uni::kStripIndex, cp)) {
    for (uint32_t i = 0; i < e[2]; ++i) out.push_back(bbh::uni::kStripData[e[1] + i]);
    return;
  }
  if (uclass(cp) != 3) out.push_back(cp);
}

void push_lower(uint32_t cp, std::vector<uint32_t>& out) {
  if (const uint32_t* e = find_map(bbh::uni::kLowerIndex, cp)) {
    for (uint32_t i = 0; i < e[2]; ++i) out.push_back(bbh::uni::kLowerData[e[1] + i]);
    return;
  }
  out.push_back(cp);
}

// UTF-8 -> code points; malformed sequences become U+FFFD (which clean_text
// then drops).
void decode_utf8(const char* s, size_t len, std::vector<uint32_t>& out) {
  const unsigned char* p = reinterpret_cast<const unsigned char*>(s);
  const unsigned char* end = p + len;
  while (p < end) {
    const unsigned c = *p;
    int n = 0;
    uint32_t cp = 0, min = 0;
    if (c < 0x80) {
      out.push_back(c);
      ++p;
      continue;
    } else if ((c & 0xE0) == 0xC0) {
      n = 1, cp = c & 0x1F, min = 0x80;
    } else if ((c & 0xF0) == 0xE0) {
      n = 2, cp = c & 0x0F, min = 0x800;
    } else if ((c & 0xF8) == 0xF0) {
      n = 3, cp = c & 0x07, min = 0x10000;
    } else {
      out.push_back(0xFFFD);
      ++p;
      continue;
    }
    int i = 1;
    for (; i <= n; ++i) {
      if (p + i >= end || (p[i] & 0xC0) != 0x80) break;
      cp = (cp << 6) | (p[i] & 0x3F);
    }
    if (i <= n || cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) {
      out.push_back(0xFFFD);
      p += (i <= n) ? i : n + 1;
      continue;
    }
    out.push_back(cp);
    p += n + 1;
  }
}

void append_utf8(uint32_t cp, std::string& s) {
  if (cp < 0x80) {
    s += (char)cp;
  } else if (cp < 0x800) {
    s += (char)(0xC0 | (cp >> 6));
    s += (char)(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    s += (char)(0xE0 | (cp >> 12));
    s += (char)(0x80 | ((cp >> 6) & 0x3F));
    s += (char)(0x80 | (cp & 0x3F));
  } else {
    s += (char)(0xF0 | (cp >> 18));
    s += (char)(0x80 | ((cp >> 12) & 0x3F));
    s += (char)(0x80 | ((cp >> 6) & 0x3F));
    s += (char)(0x80 | (cp & 0x3F));
  }
}

// WordPiece pieces of one pre-tokenized word, appended to ids.
void wordpiece(const bbh_tokenizer* t, const std::vector<uint32_t>& word, std::vector<int32_t>& ids) {
  if (word.size() > 100) {
    ids.push_back(t->unk);
    return;
  }
  std::string utf8;
  std::vector<size_t> at(word.size() + 1, 0);  // byte offset of each character
  for (size_t i = 0; i < word.size(); ++i) {
    at[i] = utf8.size();
    append_utf8(word[i], utf8);
  }
  at[word.size()] = utf8.size();
  const size_t before = ids.size();
  std::string piece;
  for (size_t start = 0; start < word.size();) {
    size_t end = word.size();
    int32_t found = -1;
    while (start < end) {
      piece.assign(start > 0 ? "##" : "");
      piece.append(utf8, at[start], at[end] - at[start]);
      auto it = t->vocab.find(piece);
      if (it != t->vocab.end()) {
        found = it->second;
        break;
      }
      --end;
    }
    if (found < 0) {  // no piece matches here: the whole word is unknown
      ids.resize(before);
      ids.push_back(t->unk);
      return;
    }
    ids.push_back(found);
    start = end;
  }
}

// Token ids of one text segment without special tokens, appended to ids.
void tokenize_segment(const bbh_tokenizer* t, const char* text, size_t len,
                      std::vector<int32_t>& ids, std::vector<uint32_t>& cps,
                      std::vector<uint32_t>& norm, std::vector<uint32_t>& tmp) {
  cps.clear();
  decode_utf8(text, len, cps);
  // clean text, CJK padding
  norm.clear();
  for (uint32_t c : cps) {
    if (c == 0 || c == 0xFFFD || is_control(c)) continue;
    if (is_whitespace(c)) {
      norm.push_back(' ');
    } else if (is_cjk(c)) {
      norm.push_back(' ');
      norm.push_back(c);
      norm.push_back(' ');
    } else {
      norm.push_back(c);
    }
  }
  if (t->lowercase) {  // accents stripped, then lowercased
    tmp.clear();
    for (uint32_t c : norm) push_stripped(c, tmp);
    norm.clear();
    for (uint32_t c : tmp) push_lower(c, norm);
  }
  // split on whitespace and punctuation, WordPiece each word
  std::vector<uint32_t> word;
  for (uint32_t c : norm) {
    if (is_whitespace(c)) {
      if (!word.empty()) wordpiece(t, word, ids);
      word.clear();
    } else if (is_punctuation(c)) {
      if (!word.empty()) wordpiece(t, word, ids);
      word.assign(1, c);
      wordpiece(t, word, ids);
      word.clear();
    } else {
      word.push_back(c);
    }
  }
  if (!word.empty()) wordpiece(t, word, ids);
}

// All token ids of one text: special tokens written verbatim ("[CLS]", ...)
// are matched first, leftmost-longest and case-sensitively, as the Hugging
// Face tokenizer does for its registered special tokens; the text between
// them is normalised and WordPiece-split.
void tokenize_text(const bbh_tokenizer* t, const char* text, std::vector<int32_t>& ids,
                   std::vector<uint32_t>& cps, std::vector<uint32_t>& norm,
                   std::vector<uint32_t>& tmp) {
  ids.clear();
  const size_t n = strlen(text);
  size_t seg = 0;
  for (size_t i = 0; i < n; ++i) {
    if (text[i] != '[') continue;
    size_t best = 0;
    int32_t id = -1;
    for (const auto& sp : t->specials)
      if (sp.first.size() > best && n - i >= sp.first.size() &&
          memcmp(text + i, sp.first.data(), sp.first.size()) == 0) {
        best = sp.first.size();
        id = sp.second;
      }
    if (id < 0) continue;
    tokenize_segment(t, text + seg, i - seg, ids, cps, norm, tmp);
    ids.push_back(id);
    i += best - 1;
    seg = i + 1;
  }
  tokenize_segment(t, text + seg, n - seg, ids, cps, norm, tmp);
}

}  // namespace

extern "C" {

bbh_status bbh_tokenizer_load(const char* vocab_path, int lowercase, bbh_tokenizer** out) {
  if (!vocab_path || !out) return set_error(BBH_ERR_INVALID_ARG, "null vocab path/out");
  *out = nullptr;
  FILE* f = fopen(vocab_path, "rb");
  if (!f) return set_error(BBH_ERR_IO, std::string("cannot open ") + vocab_path);
  auto* t = new bbh_tokenizer();
  t->lowercase = lowercase != 0;
  std::string line;
  int32_t id = 0;
  int ch;
  bool pending = false;
  auto finish = [&]() {  // one line = one token, trailing whitespace trimmed
    while (!line.empty() && (line.back() == '\r' || line.back() == ' ' || line.back() == '\t'))
      line.pop_back();
    t->vocab[line] = id++;
    line.clear();
  };
  while ((ch = fgetc(f)) != EOF) {
    pending = true;
    if (ch == '\n') {
      finish();
      pending = false;
    } else {
      line += (char)ch;
    }
  }
  if (pending) finish();
  fclose(f);
  t->size = id;
  auto special = [&](const char* name, int32_t& v) {
    auto it = t->vocab.find(name);
    v = it == t->vocab.end() ? -1 : it->second;
    return v >= 0;
  };
  if (!special("[CLS]", t->cls) || !special("[SEP]", t->sep) || !special("[PAD]", t->pad) ||
      !special("[UNK]", t->unk)) {
    delete t;
    return set_error(BBH_ERR_IO, std::string(vocab_path) +
                                     ": vocabulary lacks one of [CLS] [SEP] [PAD] [UNK]");
  }
  for (const char* name : {"[PAD]", "[UNK]", "[CLS]", "[SEP]", "[MASK]"}) {
    auto it = t->vocab.find(name);
    if (it != t->vocab.end()) t->specials.emplace_back(name, it->second);
  }
  *out = t;
  return BBH_OK;
}

bbh_status bbh_tokenizer_free(bbh_tokenizer* t) {
  delete t;
  return BBH_OK;
}

int bbh_tokenizer_vocab_size(const bbh_tokenizer* t) { return t ? t->size : 0; }

bbh_status bbh_tokenize(const bbh_tokenizer* t, const char* const* texts, int n, int seq,
                        int32_t* ids, int32_t* types, int32_t* mask, int32_t* lengths) {
  if (!t || (n > 0 && (!texts || !ids || !types || !mask)))
    return set_error(BBH_ERR_INVALID_ARG, "bbh_tokenize: null argument");
  if (n < 0 || seq < 2) return set_error(BBH_ERR_INVALID_ARG, "bbh_tokenize: n >= 0, seq >= 2");
  std::vector<int32_t> tok;
  std::vector<uint32_t> a, b, c;
  for (int i = 0; i < n; ++i) {
    if (!texts[i]) return set_error(BBH_ERR_INVALID_ARG, "bbh_tokenize: null text " + std::to_string(i));
    tokenize_text(t, texts[i], tok, a, b, c);
    const int keep = (int)tok.size() < seq - 2 ? (int)tok.size() : seq - 2;
    int32_t* row = ids + (size_t)i * seq;
    row[0] = t->cls;
    for (int j = 0; j < keep; ++j) row[1 + j] = tok[j];
    row[keep + 1] = t->sep;
    for (int j = keep + 2; j < seq; ++j) row[j] = t->pad;
    for (int j = 0; j < seq; ++j) {
      types[(size_t)i * seq + j] = 0;
      mask[(size_t)i * seq + j] = j < keep + 2 ? 1 : 0;
    }
    if (lengths) lengths[i] = keep + 2;
  }
  return BBH_OK;
}

}  // extern "C"

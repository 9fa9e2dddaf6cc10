// sg_tokenizer.cpp -- the reference's SentencePiece-style tokenizer
// (internal/tokenizer/tokenizer.go) on the host, behind the C ABI: token IDs
// for sg_forward from text, as Model.Tokenizer().Encode gives them to
// embedPrompt (pkg/ggufembed/api.go:211-234).
//
// Encode (tokenizer.go:99-133):
//   1. text as Go sees it: UTF-8 decoded rune by rune, each byte of an
//      ill-formed sequence becoming U+FFFD (what preprocessSpaces' range loop
//      writes back);
//   2. Normalize (:459-494): NFKC, then accents removed (NFD, drop Mn), then
//      per-rune simple lowercase (strings.ToLower = unicode.ToLower);
//   3. preprocessSpaces (:161-215): a lone ' ' becomes U+2581, runs of two or
//      more spaces stay raw;
//   4. tokenizeBPE (:217-348): runes are the first symbols; repeatedly merge
//      the adjacent pair whose concatenation is in the vocabulary with the
//      highest score, ties to the rightmost pair; symbols still outside the
//      vocabulary become byte tokens vocab[238 + b] when the vocabulary has
//      more than 493 entries, else vocab[unk];
//   5. strings to ids through the string -> id map (the last index of a
//      duplicated string wins, :88-91), unknown -> unk, BOS / EOS around.
// The reference rescans every pair after each merge; here the pairs sit in a
// max-heap keyed (score, left position) with lazily invalidated entries,
// which picks the same pair at every step (one pair per left position, so
// the key order is total) in O(n log n).
//
// NFKC, NFD and the character classes come from ICU (Unicode 14); the
// reference uses golang.org/x/text v0.30.0 (Unicode 15), which also inserts
// U+034F after 30 consecutive non-starters.  Texts that reach either
// difference (characters new in Unicode 15, runs of 31+ combining marks)
// may normalize differently.
#include <unicode/uchar.h>
#include <unicode/unorm2.h>
#include <unicode/ustring.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <queue>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "semantica_gpu.h"
#include "sg_internal.h"

using sgi::fail;

struct sg_tokenizer {
  sgi::TokenizerSpec spec;
  std::unordered_map<std::string, int32_t> to_id;
};

namespace {

constexpr uint32_t kReplacement = 0xFFFD;
constexpr uint32_t kMetaspace = 0x2581;
constexpr int kByteBase = 238;      // byte token of b is vocab[238 + b] (tokenizer.go:322-331)
constexpr int kByteVocabMin = 494;  // byte fallback needs len(vocab) > 493

// utf8.DecodeRune's rules: RFC 3629 sequences only (no overlongs, no
// surrogates, nothing above U+10FFFF); an invalid byte decodes as U+FFFD of
// width 1.
std::vector<uint32_t> decode_go(const char* s, size_t n) {
  std::vector<uint32_t> out;
  out.reserve(n);
  const uint8_t* p = reinterpret_cast<const uint8_t*>(s);
  size_t i = 0;
  while (i < n) {
    const uint8_t c = p[i];
    if (c < 0x80) {
      out.push_back(c);
      i++;
      continue;
    }
    int len = 0;
    uint32_t cp = 0, lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) {
      len = 2;
      cp = c & 0x1F;
    } else if (c >= 0xE0 && c <= 0xEF) {
      len = 3;
      cp = c & 0x0F;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;  // no surrogates
    } else if (c >= 0xF0 && c <= 0xF4) {
      len = 4;
      cp = c & 0x07;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    }
    bool ok = len > 0 && i + len <= n;
    for (int k = 1; ok && k < len; k++) {
      const uint8_t b = p[i + k];
      if (b < (k == 1 ? lo : 0x80) || b > (k == 1 ? hi : 0xBF)) ok = false;
      cp = (cp << 6) | (b & 0x3F);
    }
    if (ok) {
      out.push_back(cp);
      i += len;
    } else {
      out.push_back(kReplacement);
      i += 1;
    }
  }
  return out;
}

void append_utf8(std::string& s, uint32_t c) {
  if (c < 0x80) {
    s += (char)c;
  } else if (c < 0x800) {
    s += (char)(0xC0 | (c >> 6));
    s += (char)(0x80 | (c & 0x3F));
  } else if (c < 0x10000) {
    s += (char)(0xE0 | (c >> 12));
    s += (char)(0x80 | ((c >> 6) & 0x3F));
    s += (char)(0x80 | (c & 0x3F));
  } else {
    s += (char)(0xF0 | (c >> 18));
    s += (char)(0x80 | ((c >> 12) & 0x3F));
    s += (char)(0x80 | ((c >> 6) & 0x3F));
    s += (char)(0x80 | (c & 0x3F));
  }
}

// Code points -> normalized code points through one ICU normalizer.
int icu_normalize(const UNormalizer2* nz, const std::vector<uint32_t>& in, std::vector<uint32_t>& out) {
  std::vector<UChar> src;
  src.reserve(in.size() + 8);
  for (uint32_t c : in) {
    if (c < 0x10000) {
      src.push_back((UChar)c);
    } else {
      src.push_back((UChar)(0xD7C0 + (c >> 10)));
      src.push_back((UChar)(0xDC00 | (c & 0x3FF)));
    }
  }
  UErrorCode st = U_ZERO_ERROR;
  int32_t need = unorm2_normalize(nz, src.data(), (int32_t)src.size(), nullptr, 0, &st);
  if (st != U_BUFFER_OVERFLOW_ERROR && U_FAILURE(st))
    return fail(SG_ERR_INVALID, "normalization failed: %s", u_errorName(st));
  std::vector<UChar> dst((size_t)need + 1);
  st = U_ZERO_ERROR;
  need = unorm2_normalize(nz, src.data(), (int32_t)src.size(), dst.data(), (int32_t)dst.size(), &st);
  if (U_FAILURE(st)) return fail(SG_ERR_INVALID, "normalization failed: %s", u_errorName(st));
  out.clear();
  for (int32_t i = 0; i < need; i++) {
    uint32_t c = dst[i];
    if (c >= 0xD800 && c < 0xDC00 && i + 1 < need && dst[i + 1] >= 0xDC00 && dst[i + 1] < 0xE000) {
      c = 0x10000 + ((c - 0xD800) << 10) + (dst[i + 1] - 0xDC00);
      i++;
    }
    out.push_back(c);
  }
  return SG_OK;
}

// Normalizer.Normalize (tokenizer.go:459-494).
int normalize(const sgi::TokenizerSpec& sp, std::vector<uint32_t>& cps) {
  UErrorCode st = U_ZERO_ERROR;
  if (sp.nfkc) {
    const UNormalizer2* nfkc = unorm2_getNFKCInstance(&st);
    if (U_FAILURE(st)) return fail(SG_ERR_INVALID, "NFKC unavailable: %s", u_errorName(st));
    std::vector<uint32_t> t;
    SG_TRY(icu_normalize(nfkc, cps, t));
    cps.swap(t);
  }
  if (sp.remove_accents) {
    const UNormalizer2* nfd = unorm2_getNFDInstance(&st);
    if (U_FAILURE(st)) return fail(SG_ERR_INVALID, "NFD unavailable: %s", u_errorName(st));
    std::vector<uint32_t> t;
    SG_TRY(icu_normalize(nfd, cps, t));
    cps.clear();
    for (uint32_t c : t)
      if (u_charType((UChar32)c) != U_NON_SPACING_MARK) cps.push_back(c);
  }
  if (sp.lowercase)
    for (uint32_t& c : cps) c = (uint32_t)u_tolower((UChar32)c);
  return SG_OK;
}

// preprocessSpaces (tokenizer.go:161-215): the symbols' initial texts.
std::vector<std::string> preprocess(const std::vector<uint32_t>& cps) {
  std::vector<std::string> sym;
  sym.reserve(cps.size());
  size_t i = 0;
  while (i < cps.size()) {
    if (cps[i] != ' ') {
      std::string t;
      append_utf8(t, cps[i]);
      sym.push_back(std::move(t));
      i++;
      continue;
    }
    size_t j = i;
    while (j < cps.size() && cps[j] == ' ') j++;
    if (j - i == 1) {
      std::string t;
      append_utf8(t, kMetaspace);
      sym.push_back(std::move(t));
    } else {
      for (size_t k = i; k < j; k++) sym.push_back(" ");
    }
    i = j;
  }
  return sym;
}

struct Pair {
  float score;
  int left, right;
  uint32_t ver_l, ver_r;
  bool operator<(const Pair& o) const {  // max-heap on (score, left)
    return score < o.score || (score == o.score && left < o.left);
  }
};

// tokenizeBPE (tokenizer.go:217-348) -> final token strings.
std::vector<std::string> bpe(const sg_tokenizer* t, std::vector<std::string> text) {
  const int n = (int)text.size();
  std::vector<int> prev(n), next(n);
  std::vector<uint32_t> ver(n, 0);
  for (int i = 0; i < n; i++) {
    prev[i] = i - 1;
    next[i] = i + 1 < n ? i + 1 : -1;
  }
  std::priority_queue<Pair> heap;
  auto add = [&](int l, int r) {
    if (l < 0 || r < 0) return;
    auto it = t->to_id.find(text[l] + text[r]);
    if (it != t->to_id.end()) heap.push(Pair{t->spec.scores[it->second], l, r, ver[l], ver[r]});
  };
  for (int i = 0; i + 1 < n; i++) add(i, i + 1);
  while (!heap.empty()) {
    const Pair p = heap.top();
    heap.pop();
    if (text[p.left].empty() || next[p.left] != p.right || ver[p.left] != p.ver_l || ver[p.right] != p.ver_r)
      continue;  // stale: one side has changed since the pair was pushed
    text[p.left] += text[p.right];
    ver[p.left]++;
    next[p.left] = next[p.right];
    if (next[p.right] != -1) prev[next[p.right]] = p.left;
    text[p.right].clear();
    ver[p.right]++;
    add(prev[p.left], p.left);
    add(p.left, next[p.left]);
  }
  std::vector<std::string> out;
  const auto& vocab = t->spec.tokens;
  const bool bytes = vocab.size() > (size_t)(kByteVocabMin - 1);
  for (int i = 0; i < n; i++) {
    if (text[i].empty()) continue;
    if (t->to_id.count(text[i])) {
      out.push_back(std::move(text[i]));
    } else if (bytes) {
      for (unsigned char b : text[i]) out.push_back(vocab[kByteBase + b]);
    } else if (t->spec.unk >= 0 && t->spec.unk < (int32_t)vocab.size()) {
      out.push_back(vocab[t->spec.unk]);
    }
  }
  return out;
}

int encode(const sg_tokenizer* t, const char* text, size_t len, std::vector<int32_t>& ids) {
  std::vector<uint32_t> cps = decode_go(text, len);
  SG_TRY(normalize(t->spec, cps));
  ids.clear();
  if (t->spec.add_bos && t->spec.bos >= 0) ids.push_back(t->spec.bos);
  if (!cps.empty()) {
    for (const std::string& tok : bpe(t, preprocess(cps))) {
      auto it = t->to_id.find(tok);
      if (it != t->to_id.end())
        ids.push_back(it->second);
      else if (t->spec.unk >= 0)
        ids.push_back(t->spec.unk);
    }
  }
  if (t->spec.add_eos && t->spec.eos >= 0) ids.push_back(t->spec.eos);
  return SG_OK;
}

// tokenizer.New (:56-97) checks + the string -> id map.
int make_tokenizer(sgi::TokenizerSpec&& sp, sg_tokenizer** out) {
  if (sp.tokens.size() != sp.scores.size())
    return fail(SG_ERR_INVALID, "vocab and scores length mismatch: %zu != %zu", sp.tokens.size(), sp.scores.size());
  if (!sp.types.empty() && sp.types.size() != sp.tokens.size())
    return fail(SG_ERR_INVALID, "vocab and tokenTypes length mismatch: %zu != %zu", sp.tokens.size(),
                sp.types.size());
  if (sp.types.empty()) sp.types.assign(sp.tokens.size(), 1);
  sg_tokenizer* t = new sg_tokenizer;
  t->spec = std::move(sp);
  t->to_id.reserve(t->spec.tokens.size());
  for (size_t i = 0; i < t->spec.tokens.size(); i++) t->to_id[t->spec.tokens[i]] = (int32_t)i;
  *out = t;
  return SG_OK;
}

}  // namespace

extern "C" {

int sg_tokenizer_create(const char* token_data, const int64_t* token_offsets, const float* scores,
                        const int32_t* token_types, int32_t n, const sg_tokenizer_config* cfg, sg_tokenizer** out) {
  if (!out || !cfg || n < 0 || (n > 0 && (!token_data || !token_offsets || !scores)))
    return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  sgi::TokenizerSpec sp;
  sp.tokens.reserve((size_t)n);
  for (int32_t i = 0; i < n; i++) {
    if (token_offsets[i + 1] < token_offsets[i]) return fail(SG_ERR_INVALID, "token offsets must not decrease");
    sp.tokens.emplace_back(token_data + token_offsets[i], (size_t)(token_offsets[i + 1] - token_offsets[i]));
  }
  sp.scores.assign(scores, scores + n);
  if (token_types) sp.types.assign(token_types, token_types + n);
  sp.add_bos = cfg->add_bos != 0;
  sp.add_eos = cfg->add_eos != 0;
  sp.lowercase = cfg->lowercase != 0;
  sp.remove_accents = cfg->remove_accents != 0;
  sp.nfkc = cfg->nfkc != 0;
  sp.bos = cfg->bos_id;
  sp.eos = cfg->eos_id;
  sp.unk = cfg->unk_id;
  sp.pad = cfg->pad_id;
  return make_tokenizer(std::move(sp), out);
}

int sg_tokenizer_from_gguf(const void* data, size_t size, sg_tokenizer** out) {
  if (!out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  sgi::TokenizerSpec sp;
  SG_TRY(sgi::gguf_tokenizer_spec(data, size, sp));
  return make_tokenizer(std::move(sp), out);
}

int sg_tokenizer_encode(const sg_tokenizer* t, const char* text, size_t len, int32_t* ids, int32_t cap,
                        int32_t* n_ids) {
  if (!t || !n_ids || (!text && len)) return fail(SG_ERR_INVALID, "NULL argument");
  std::vector<int32_t> v;
  SG_TRY(encode(t, text ? text : "", len, v));
  *n_ids = (int32_t)v.size();
  if (ids && cap > 0) memcpy(ids, v.data(), sizeof(int32_t) * std::min<size_t>(v.size(), (size_t)cap));
  return SG_OK;
}

int sg_tokenizer_encode_batch(const sg_tokenizer* t, const char* text_data, const int64_t* text_offsets,
                              int32_t n_texts, int32_t* ids, int64_t cap, int32_t* id_offsets) {
  if (!t || !id_offsets || n_texts < 0 || (n_texts > 0 && (!text_data || !text_offsets)))
    return fail(SG_ERR_INVALID, "NULL argument");
  for (int32_t i = 0; i < n_texts; i++)
    if (text_offsets[i + 1] < text_offsets[i]) return fail(SG_ERR_INVALID, "text offsets must not decrease");
  // Texts are independent: contiguous ranges of them go to worker threads
  // (the ICU normalizers are immutable shared instances).
  std::vector<std::vector<int32_t>> res((size_t)n_texts);
  const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
  const int workers = std::max(1, std::min(hw, n_texts / 4));
  std::vector<int> rc((size_t)workers, SG_OK);
  std::vector<std::string> msg((size_t)workers);
  auto run = [&](int w) {
    const int32_t b = (int32_t)((int64_t)n_texts * w / workers), e = (int32_t)((int64_t)n_texts * (w + 1) / workers);
    for (int32_t i = b; i < e && rc[w] == SG_OK; i++) {
      rc[w] = encode(t, text_data + text_offsets[i], (size_t)(text_offsets[i + 1] - text_offsets[i]), res[i]);
      if (rc[w] != SG_OK) msg[w] = sg_last_error();  // the message is thread-local
    }
  };
  if (workers == 1) {
    run(0);
  } else {
    std::vector<std::thread> th;
    for (int w = 0; w < workers; w++) th.emplace_back(run, w);
    for (auto& x : th) x.join();
  }
  for (int w = 0; w < workers; w++)
    if (rc[w] != SG_OK) return fail(rc[w], "%s", msg[w].c_str());
  id_offsets[0] = 0;
  int64_t pos = 0;
  for (int32_t i = 0; i < n_texts; i++) {
    const auto& v = res[i];
    if (pos + (int64_t)v.size() > INT32_MAX) return fail(SG_ERR_INVALID, "more than 2^31 token IDs");
    if (ids && pos + (int64_t)v.size() <= cap) memcpy(ids + pos, v.data(), sizeof(int32_t) * v.size());
    pos += (int64_t)v.size();
    id_offsets[i + 1] = (int32_t)pos;
  }
  if (ids && pos > cap) return fail(SG_ERR_INVALID, "ids buffer of %lld, %lld needed", (long long)cap, (long long)pos);
  return SG_OK;
}

int sg_tokenizer_decode(const sg_tokenizer* t, const int32_t* ids, int32_t n, char* buf, size_t cap, size_t* len) {
  if (!t || !len || (!ids && n > 0)) return fail(SG_ERR_INVALID, "NULL argument");
  // Decode (tokenizer.go:135-159): out-of-range and special ids skipped,
  // U+2581 -> ' ' in every token.
  const auto& sp = t->spec;
  std::string s;
  for (int32_t k = 0; k < n; k++) {
    const int32_t id = ids[k];
    if (id < 0 || id >= (int32_t)sp.tokens.size()) continue;
    if (id == sp.bos || id == sp.eos || id == sp.unk || id == sp.pad || sp.types[id] == 3 || sp.types[id] == 5)
      continue;
    const std::string& tok = sp.tokens[id];
    for (size_t i = 0; i < tok.size();) {
      if (i + 2 < tok.size() && (uint8_t)tok[i] == 0xE2 && (uint8_t)tok[i + 1] == 0x96 && (uint8_t)tok[i + 2] == 0x81) {
        s += ' ';
        i += 3;
      } else {
        s += tok[i++];
      }
    }
  }
  *len = s.size();
  if (buf && cap) memcpy(buf, s.data(), std::min(cap, s.size()));
  return SG_OK;
}

int32_t sg_tokenizer_vocab_size(const sg_tokenizer* t) { return t ? (int32_t)t->spec.tokens.size() : 0; }

void sg_tokenizer_free(sg_tokenizer* t) { delete t; }

}  // extern "C"

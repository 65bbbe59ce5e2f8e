// Host sanitizer check of the safetensors / JSON reader: a valid teeny-quant
// style image, then many deterministic mutations of it (byte flips, header
// length edits, truncations, spliced JSON tokens).  Every open must return
// (true or false) without a sanitizer report; the valid image must parse.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../teenygrad_amd/csrc/safetensors.hpp"

using teeny::st::File;

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next() {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}

static std::vector<uint8_t> image(const std::string &header, size_t data_bytes) {
  std::vector<uint8_t> v(8 + header.size() + data_bytes, 0);
  uint64_t n = header.size();
  for (int i = 0; i < 8; ++i) v[i] = static_cast<uint8_t>(n >> (8 * i));
  std::memcpy(v.data() + 8, header.data(), header.size());
  for (size_t i = 0; i < data_bytes; ++i) v[8 + header.size() + i] = static_cast<uint8_t>(i * 7);
  return v;
}

int main() {
  const std::string cfg =
      "{\\\"quant_method\\\":\\\"compressed-tensors\\\",\\\"format\\\":\\\"int-quantized\\\",\\\"config_groups\\\":"
      "{\\\"group_0\\\":{\\\"weights\\\":{\\\"num_bits\\\":8,\\\"type\\\":\\\"int\\\",\\\"symmetric\\\":true,"
      "\\\"strategy\\\":\\\"channel\\\",\\\"axis\\\":0},\\\"targets\\\":[\\\"*\\\"]}},\\\"ignore\\\":[\\\"fc.bias\\\"]}";
  const std::string header = "{\"__metadata__\":{\"quantization_config\":\"" + cfg +
                             "\"},\"fc.bias\":{\"dtype\":\"F32\",\"shape\":[4],\"data_offsets\":[0,16]},"
                             "\"fc.weight\":{\"dtype\":\"I8\",\"shape\":[4,8],\"data_offsets\":[16,48]},"
                             "\"fc.weight_scale\":{\"dtype\":\"F32\",\"shape\":[4],\"data_offsets\":[48,64]},"
                             "\"u\":{\"dtype\":\"I8\",\"shape\":[2],\"data_offsets\":[64,66],\"x\":\"\\u00e9\\ud83d\\ude00\"}}";
  const std::vector<uint8_t> good = image(header, 66);
  {
    File f;
    std::string err;
    if (!f.open_image(good.data(), good.size(), &err) || f.tensors().size() != 4 || !f.quant_config().present ||
        f.quant_config().axis != 0 || f.quant_config().ignore.size() != 1) {
      std::fprintf(stderr, "valid image rejected: %s\n", err.c_str());
      return 1;
    }
  }
  const char *tokens[] = {"{", "}", "[", "]", "\"", ":", ",", "-", "1e999", "99999999999999999999", "\\u", "\\ud800",
                          "null", "true", "\"dtype\"", "\"shape\"", "\"data_offsets\"", "[0,1]", "\x01", "\xff"};
  int ok = 0, rejected = 0;
  for (int iter = 0; iter < 20000; ++iter) {
    std::vector<uint8_t> m = good;
    const int kind = static_cast<int>(next() % 5);
    if (kind == 0) {  // flip bytes
      for (int k = 0; k < 1 + static_cast<int>(next() % 4); ++k) m[next() % m.size()] ^= static_cast<uint8_t>(1u << (next() % 8));
    } else if (kind == 1) {  // edit the header length
      uint64_t n = next() % (m.size() + 64);
      for (int i = 0; i < 8; ++i) m[i] = static_cast<uint8_t>(n >> (8 * i));
    } else if (kind == 2) {  // truncate
      m.resize(next() % m.size());
    } else if (kind == 3) {  // splice a JSON token into the header
      std::string h = header;
      const char *t = tokens[next() % (sizeof(tokens) / sizeof(tokens[0]))];
      h.insert(next() % (h.size() + 1), t);
      m = image(h, 66);
    } else {  // delete a span of the header
      std::string h = header;
      const size_t at = next() % h.size();
      h.erase(at, 1 + next() % 16);
      m = image(h, 66);
    }
    // an exact-size heap copy, so any read past its end is caught
    std::vector<uint8_t> exact(m.begin(), m.end());
    File f;
    std::string err;
    const uint8_t *p = exact.empty() ? nullptr : exact.data();
    if (f.open_image(p, exact.size(), &err)) {
      ++ok;
      for (const auto &t : f.tensors()) {  // touch every tensor's bytes
        const uint8_t *d = f.data(t);
        volatile uint8_t acc = 0;
        for (uint64_t i = 0; i < t.end - t.begin; ++i) acc ^= d[i];
        (void)acc;
      }
    } else {
      ++rejected;
    }
  }
  // the JSON parser alone on nested and numeric edge cases
  const char *docs[] = {"[[[[[[[[]]]]]]]]", "{\"a\":[1,2.5,-0,1e3,true,false,null,\"x\"]}", "-", "01", "1.", "1e",
                        "\"\\uD83D\\uDE00\"", "\"\\uDE00\"", "{\"a\" 1}", "[1,]", "9223372036854775808"};
  for (const char *d : docs) {
    teeny::st::Json j;
    std::string err;
    teeny::st::parse_json(d, std::strlen(d), &j, &err);
  }
  std::printf("fuzz: %d accepted, %d rejected\n", ok, rejected);
  return 0;
}

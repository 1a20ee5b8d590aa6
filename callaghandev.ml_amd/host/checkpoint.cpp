// Checkpoint directory of LanguageModel.Save / Load (LanguageModel.cs:706-919):
//
//   config.json             the configuration dictionary of Save (:710-735),
//                           System.Text.Json, indented
//   weights.bin             a BinaryWriter stream (:737-765): one bool byte
//                           (discrete tokens), then matrices as int32 rows,
//                           int32 cols and rows*cols float32 row-major, and
//                           vectors as int32 length and float32 values, all
//                           little-endian.  Order: TokenEmbedding or
//                           InputProjection + InputProjectionBias; per block
//                           WQ WK WV WO BiasQ BiasK BiasV BiasO (:865-869),
//                           LN1Gamma LN1Beta LN2Gamma LN2Beta; OutputProjection,
//                           OutputBias
//   ffn/ffn_layer_<i>.json  block i's FFN NeuralNetwork (:671-705), the
//                           Newtonsoft.Json form of Neural Network/Data.cs
//                           (:218-257): {"layers": [Layer...], "parameters":
//                           {...}}, a Layer holding Size, InputSize,
//                           Activations, Biases, Derivatives, Deltas, Weights
//                           [Size][InputSize] and ActivationType
//
// Load follows the reference's checks and messages: shape mismatches raise
// InvalidOperationException with the reference's text (:871-904), a missing
// FFN file FileNotFoundException, a truncated weights.bin the text of .NET's
// EndOfStreamException.  A missing config key (KeyNotFoundException in the
// reference) raises InvalidOperationException naming the key.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <sstream>

#include "cdml_host.h"

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "weights.bin is little-endian");

namespace cdml_host {
namespace {

namespace fs = std::filesystem;

std::string read_file(const fs::path &p) {
  std::ifstream f(p, std::ios::binary);
  if (!f) throw FileNotFoundException("Could not find file '" + p.string() + "'.");
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

void write_file(const fs::path &p, const std::string &bytes) {
  std::ofstream f(p, std::ios::binary | std::ios::trunc);
  if (!f) throw InvalidOperationException("Could not open '" + p.string() + "' for writing.");
  f.write(bytes.data(), (std::streamsize)bytes.size());
  if (!f) throw InvalidOperationException("Could not write '" + p.string() + "'.");
}

// ---- JSON ------------------------------------------------------------------
// A pull reader over the whole text: the caller walks the structure it
// expects and skips the rest, so a multi-million-element weight array is read
// straight into floats without an intermediate tree.
class JsonReader {
 public:
  JsonReader(const std::string &text, std::string name) : s_(text), name_(std::move(name)) {
    if (s_.compare(0, 3, "\xEF\xBB\xBF") == 0) i_ = 3;  // UTF-8 byte-order mark
  }
  char peek() {
    ws();
    return i_ < s_.size() ? s_[i_] : '\0';
  }
  void expect(char c) {
    if (peek() != c) fail(std::string("expected '") + c + "'");
    ++i_;
  }
  bool consume(char c) {
    if (peek() != c) return false;
    ++i_;
    return true;
  }
  bool null() {
    ws();
    return match("null");
  }
  std::string str() {
    expect('"');
    std::string out;
    while (true) {
      if (i_ >= s_.size()) fail("unterminated string");
      const char c = s_[i_++];
      if (c == '"') return out;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) fail("unterminated escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': case '\\': case '/': out += e; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          if (i_ + 4 > s_.size()) fail("short \\u escape");
          const unsigned cp = (unsigned)std::strtoul(s_.substr(i_, 4).c_str(), nullptr, 16);
          i_ += 4;
          if (cp < 0x80) {
            out += (char)cp;
          } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
          } else {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
          }
          break;
        }
        default: fail("bad escape");
      }
    }
  }
  std::string number_token() {
    ws();
    const size_t b = i_;
    while (i_ < s_.size() && std::strchr("+-0123456789.eE", s_[i_]) && s_[i_] != '\0') ++i_;
    if (b == i_) fail("expected a number");
    return s_.substr(b, i_ - b);
  }
  double number() {
    const std::string t = number_token();
    char *end = nullptr;
    const double v = std::strtod(t.c_str(), &end);
    if (*end) fail("bad number '" + t + "'");
    return v;
  }
  int int32() {
    const double v = number();
    if (v != std::floor(v) || v < -2147483648.0 || v > 2147483647.0) fail("expected a 32-bit integer");
    return (int)v;
  }
  // A float32 element: a number (converted once, decimal -> float, so a
  // shortest round-trip string gives back the saved float), or Newtonsoft's
  // string forms of the non-finite values.
  float f32() {
    if (peek() == '"') {
      const std::string t = str();
      if (t == "NaN") return NAN;
      if (t == "Infinity") return INFINITY;
      if (t == "-Infinity") return -INFINITY;
      fail("bad float '" + t + "'");
    }
    const std::string t = number_token();
    char *end = nullptr;
    const float v = std::strtof(t.c_str(), &end);
    if (*end) fail("bad number '" + t + "'");
    return v;
  }
  bool boolean() {
    ws();
    if (match("true")) return true;
    if (match("false")) return false;
    fail("expected true or false");
  }
  template <class F>
  void object(F &&on_key) {
    expect('{');
    if (consume('}')) return;
    do {
      const std::string k = str();
      expect(':');
      on_key(k);
    } while (consume(','));
    expect('}');
  }
  template <class F>
  void array(F &&on_elem) {
    expect('[');
    if (consume(']')) return;
    do on_elem();
    while (consume(','));
    expect(']');
  }
  void skip() {
    const char c = peek();
    if (c == '{') {
      object([&](const std::string &) { skip(); });
    } else if (c == '[') {
      array([&] { skip(); });
    } else if (c == '"') {
      str();
    } else if (!(match("true") || match("false") || match("null"))) {
      number_token();
    }
  }
  void end() {
    if (peek() != '\0') fail("unexpected content after the document");
  }
  [[noreturn]] void fail(const std::string &what) {
    throw InvalidOperationException(name_ + ": " + what + " at byte " + std::to_string(i_) + ".");
  }

 private:
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  bool match(const char *lit) {
    const size_t n = std::strlen(lit);
    if (s_.compare(i_, n, lit) != 0) return false;
    i_ += n;
    return true;
  }
  const std::string &s_;
  std::string name_;
  size_t i_ = 0;
};

// Shortest decimal that reads back as the same float, with a decimal point
// as Newtonsoft writes floats (EnsureDecimalPlace); non-finite values as its
// quoted strings.
std::string float_text(float v, bool ensure_point) {
  if (std::isnan(v)) return "\"NaN\"";
  if (std::isinf(v)) return v > 0 ? "\"Infinity\"" : "\"-Infinity\"";
  char buf[48];
  for (int prec = 1; prec <= 9; ++prec) {
    std::snprintf(buf, sizeof buf, "%.*g", prec, (double)v);
    if (std::strtof(buf, nullptr) == v) break;
  }
  std::string t = buf;
  if (ensure_point && t.find_first_of(".eEn") == std::string::npos) t += ".0";
  return t;
}

// ActivationType as Newtonsoft writes enums (an integer), also accepting the
// member names.
int activation_value(JsonReader &r) {
  if (r.peek() != '"') return r.int32();
  static const char *names[] = {"None", "Sigmoid", "Tanh", "Relu", "Leakyrelu", "Swish"};
  const std::string t = r.str();
  for (int i = 0; i < 6; ++i)
    if (t == names[i]) return i;
  r.fail("unknown ActivationType '" + t + "'");
}

struct FfnLayer {
  int size = -1;
  int act = 0;
  Matrix w;  // [size, input]
  std::vector<float> b;
  bool has_w = false, has_b = false;
};

FfnLayer read_ffn_layer(JsonReader &r) {
  FfnLayer L;
  r.object([&](const std::string &k) {
    if (k == "Weights") {
      if (r.null()) return;
      L.has_w = true;
      int rows = 0, cols = -1;
      std::vector<float> flat;
      r.array([&] {
        size_t before = flat.size();
        r.array([&] { flat.push_back(r.f32()); });
        const int n = (int)(flat.size() - before);
        if (cols < 0) cols = n;
        else if (n != cols) r.fail("Weights rows differ in length");
        ++rows;
      });
      L.w.rows = rows;
      L.w.cols = cols < 0 ? 0 : cols;
      L.w.data.assign(flat.begin(), flat.end());
    } else if (k == "Biases") {
      if (r.null()) return;
      L.has_b = true;
      r.array([&] { L.b.push_back(r.f32()); });
    } else if (k == "ActivationType") {
      L.act = activation_value(r);
    } else if (k == "Size") {
      L.size = r.int32();
    } else {
      r.skip();
    }
  });
  return L;
}

// NeuralNetwork.Load of one FFN file followed by RestoreState (:692-703):
// the file's layers replace the network.
FeedForwardNetwork read_ffn(const fs::path &p) {
  const std::string text = read_file(p);
  JsonReader r(text, p.string());
  std::vector<FfnLayer> layers;
  bool have_layers = false;
  r.object([&](const std::string &k) {
    if (k == "layers") {
      have_layers = true;
      if (r.null()) r.fail("layers is null");
      r.array([&] { layers.push_back(read_ffn_layer(r)); });
    } else {
      r.skip();
    }
  });
  r.end();
  if (!have_layers || layers.size() < 2)
    throw InvalidOperationException("Neural network must have at least input and output layers.");
  FeedForwardNetwork ffn;
  int width = layers[0].has_b ? (int)layers[0].b.size() : layers[0].size;
  for (size_t i = 1; i < layers.size(); ++i) {
    FfnLayer &L = layers[i];
    const std::string where = p.string() + ": layer " + std::to_string(i);
    if (!L.has_w || !L.has_b) throw InvalidOperationException(where + " has no Weights or Biases.");
    if (L.w.rows != (int)L.b.size() || (L.w.rows > 0 && L.w.cols != width))
      throw InvalidOperationException(where + ": Weights [" + std::to_string(L.w.rows) + "," +
                                      std::to_string(L.w.cols) + "] do not map width " +
                                      std::to_string(width) + " to " + std::to_string(L.b.size()) + ".");
    if (L.act < None || L.act > Swish) throw InvalidOperationException(where + ": bad ActivationType.");
    width = (int)L.b.size();
    ffn.weights.push_back(std::move(L.w));
    ffn.biases.push_back(std::move(L.b));
    ffn.activations.push_back(L.act);
  }
  return ffn;
}

// Data.Save (Data.cs:218-236) of a transformer FFN: Newtonsoft's indented
// layout with a UTF-8 byte-order mark (StreamWriter over Encoding.UTF8).
// The parameters are those TransformerBlock gives the FFN
// (TransformerBlock.cs:101-121).
std::string ffn_json(const FeedForwardNetwork &ffn, const TransformerConfig &c) {
  std::string o = "\xEF\xBB\xBF{\n  \"layers\": [\n";
  const int nl = (int)ffn.weights.size() + 1;
  std::vector<int> widths{ffn.input_size()};
  std::vector<int> acts{None};
  for (size_t i = 0; i < ffn.weights.size(); ++i) {
    widths.push_back(ffn.weights[i].rows);
    acts.push_back(ffn.activations[i]);
  }
  auto vec = [&](const std::string &ind, const float *v, int n) {
    if (n == 0) return std::string("[]");
    std::string t = "[\n";
    for (int i = 0; i < n; ++i) {
      t += ind + "  " + float_text(v[i], true);
      t += i + 1 < n ? ",\n" : "\n";
    }
    return t + ind + "]";
  };
  for (int li = 0; li < nl; ++li) {
    const int size = widths[li], in = li == 0 ? 0 : widths[li - 1];
    const std::vector<float> zeros(size, 0.f);
    const float *bias = li == 0 ? zeros.data() : ffn.biases[li - 1].data();
    o += "    {\n";
    o += "      \"Size\": " + std::to_string(size) + ",\n";
    o += "      \"InputSize\": " + std::to_string(in) + ",\n";
    o += "      \"Activations\": " + vec("      ", zeros.data(), size) + ",\n";
    o += "      \"Biases\": " + vec("      ", bias, size) + ",\n";
    o += "      \"Derivatives\": " + vec("      ", zeros.data(), size) + ",\n";
    o += "      \"Deltas\": " + vec("      ", zeros.data(), size) + ",\n";
    o += "      \"Weights\": ";
    if (size == 0) {
      o += "[]";
    } else {
      o += "[\n";
      for (int r = 0; r < size; ++r) {
        o += "        " + (li == 0 ? std::string("[]") : vec("        ", ffn.weights[li - 1].ptr() + (size_t)r * in, in));
        o += r + 1 < size ? ",\n" : "\n";
      }
      o += "      ]";
    }
    o += ",\n      \"ActivationType\": " + std::to_string(acts[li]) + "\n";
    o += li + 1 < nl ? "    },\n" : "    }\n";
  }
  auto ints = [](const std::vector<int> &v) {
    std::string t = "[\n";
    for (size_t i = 0; i < v.size(); ++i) t += "      " + std::to_string(v[i]) + (i + 1 < v.size() ? ",\n" : "\n");
    return t + "    ]";
  };
  const int D = ffn.input_size();
  const std::vector<float> mins(D, 0.f), maxs(D, 1.f);
  o += "  ],\n  \"parameters\": {\n";
  o += "    \"HuberLossDelta\": 1.0,\n";
  o += "    \"AccelerationType\": " + std::to_string(c.AccelerationType) + ",\n";
  o += "    \"AccelerationDeviceId\": " + std::to_string(c.AccelerationDeviceId) + ",\n";
  o += "    \"CostFunction\": " + std::to_string(c.CostFunction) + ",\n";
  o += "    \"ActivationDistribution\": " + std::to_string(c.ActivationDistribution) + ",\n";
  o += "    \"L2RegulationLamda\": " + float_text(c.L2RegulationLamda, true) + ",\n";
  o += "    \"GradientClippingThreshold\": " + float_text(c.GradientClippingThreshold, true) + ",\n";
  o += "    \"GradientExplosionThreshold\": 1000.0,\n";
  o += "    \"GradientVanishingThreshold\": 1E-05,\n";
  o += "    \"LayerWidths\": " + ints(widths) + ",\n";
  o += "    \"LayerActivations\": " + ints(acts) + ",\n";
  o += "    \"inputActivationMin\": " + vec("    ", mins.data(), D) + ",\n";
  o += "    \"inputActivationMax\": " + vec("    ", maxs.data(), D) + ",\n";
  o += "    \"OptimalLearningRate\": null,\n";
  o += "    \"EpochsTrainedOn\": 10\n";
  o += "  }\n}";
  return o;
}

// ---- weights.bin -------------------------------------------------------------
class BinReader {
 public:
  BinReader(const std::string &b, std::string name) : b_(b), name_(std::move(name)) {}
  bool boolean() {  // BinaryReader.ReadBoolean: any non-zero byte is true
    need(1);
    return b_[i_++] != 0;
  }
  int32_t i32() {
    need(4);
    int32_t v;
    std::memcpy(&v, b_.data() + i_, 4);
    i_ += 4;
    return v;
  }
  void f32(float *dst, size_t n) {
    need(4 * n);
    std::memcpy(dst, b_.data() + i_, 4 * n);
    i_ += 4 * n;
  }
  // ReadMatrixInto / ReadVectorInto (LanguageModel.cs:871-904)
  void matrix_into(Matrix &m) {
    const int rows = i32(), cols = i32();
    if (rows != m.rows || cols != m.cols)
      throw InvalidOperationException("Matrix shape mismatch. File has [" + std::to_string(rows) + "," +
                                      std::to_string(cols) + "], target is [" + std::to_string(m.rows) +
                                      "," + std::to_string(m.cols) + "].");
    f32(m.ptr(), (size_t)rows * cols);
  }
  void vector_into(std::vector<float> &v) {
    const int len = i32();
    if (len != (int)v.size())
      throw InvalidOperationException("Vector length mismatch. File has [" + std::to_string(len) +
                                      "], target is [" + std::to_string(v.size()) + "].");
    f32(v.data(), v.size());
  }

 private:
  void need(size_t n) {
    if (b_.size() - i_ < n) throw InvalidOperationException(name_ + ": Unable to read beyond the end of the stream.");
  }
  const std::string &b_;
  std::string name_;
  size_t i_ = 0;
};

struct BinWriter {
  std::string out;
  void boolean(bool v) { out += (char)(v ? 1 : 0); }
  void i32(int32_t v) { out.append(reinterpret_cast<const char *>(&v), 4); }
  void f32(const float *p, size_t n) { out.append(reinterpret_cast<const char *>(p), 4 * n); }
  void matrix(const Matrix &m) {
    i32(m.rows);
    i32(m.cols);
    f32(m.ptr(), (size_t)m.rows * m.cols);
  }
  void vector(const std::vector<float> &v) {
    i32((int32_t)v.size());
    f32(v.data(), v.size());
  }
};

// ---- config.json -------------------------------------------------------------
struct ConfigValue {
  enum Kind { Number, Bool, String, Null, Other } kind = Other;
  std::string text;
  bool flag = false;
};

std::map<std::string, ConfigValue> read_config_values(const fs::path &p) {
  const std::string text = read_file(p);
  JsonReader r(text, p.string());
  std::map<std::string, ConfigValue> vals;
  r.object([&](const std::string &k) {
    ConfigValue v;
    const char c = r.peek();
    if (c == '"') {
      v.kind = ConfigValue::String;
      v.text = r.str();
    } else if (c == 't' || c == 'f') {
      v.kind = ConfigValue::Bool;
      v.flag = r.boolean();
    } else if (c == 'n') {
      r.null();
      v.kind = ConfigValue::Null;
    } else if (c == '{' || c == '[') {
      r.skip();
    } else {
      v.kind = ConfigValue::Number;
      v.text = r.number_token();
    }
    vals[k] = v;
  });
  r.end();
  return vals;
}

}  // namespace

void LanguageModel::Save(const std::string &directory) const {
  const fs::path dir(directory);
  std::error_code ec;
  fs::create_directories(dir, ec);
  if (ec) throw InvalidOperationException("Could not create '" + directory + "': " + ec.message());
  const TransformerConfig &c = cfg_;
  // DataType as the config states it, unless it contradicts the token mode.
  const bool discrete_type = c.DataType == 0 || c.DataType == 3;
  const int data_type = discrete_type == c.UsesDiscreteTokens ? c.DataType : (c.UsesDiscreteTokens ? 0 : 1);
  std::string js = "{\n";
  auto kv = [&](const char *k, const std::string &v, bool last = false) {
    js += std::string("  \"") + k + "\": " + v + (last ? "\n" : ",\n");
  };
  kv("VocabSize", std::to_string(c.VocabSize));
  kv("MaxSequenceLength", std::to_string(c.MaxSequenceLength));
  kv("EmbeddingDim", std::to_string(c.EmbeddingDim));
  kv("NumHeads", std::to_string(c.NumHeads));
  kv("NumLayers", std::to_string(c.NumLayers));
  kv("FeedForwardDim", std::to_string(c.FeedForwardDim));
  kv("UseDecoderOnly", c.UseDecoderOnly ? "true" : "false");
  kv("FFNActivationType", std::to_string(c.FFNActivationType));
  kv("AccelerationType", std::to_string(c.AccelerationType));
  kv("AccelerationDeviceId", std::to_string(c.AccelerationDeviceId));
  kv("L2RegulationLamda", float_text(c.L2RegulationLamda, false));
  kv("GradientClippingThreshold", float_text(c.GradientClippingThreshold, false));
  kv("DataType", std::to_string(data_type));
  kv("InputFeatureDim", std::to_string(c.InputFeatureDim));
  kv("OutputDim", std::to_string(c.OutputDim));
  kv("CostFunction", std::to_string(c.CostFunction));
  kv("ActivationDistribution", std::to_string(c.ActivationDistribution), true);
  js += "}";
  write_file(dir / "config.json", js);

  BinWriter w;
  w.boolean(c.UsesDiscreteTokens);
  if (c.UsesDiscreteTokens) {
    w.matrix(TokenEmbedding);
  } else {
    w.matrix(InputProjection);
    w.vector(InputProjectionBias);
  }
  for (const TransformerBlock &b : Blocks) {
    const MultiHeadAttention &a = b.Attention;
    w.matrix(a.WQ);
    w.matrix(a.WK);
    w.matrix(a.WV);
    w.matrix(a.WO);
    w.vector(a.BiasQ);
    w.vector(a.BiasK);
    w.vector(a.BiasV);
    w.vector(a.BiasO);
    w.vector(b.LN1Gamma);
    w.vector(b.LN1Beta);
    w.vector(b.LN2Gamma);
    w.vector(b.LN2Beta);
  }
  w.matrix(OutputProjection);
  w.vector(OutputBias);
  write_file(dir / "weights.bin", w.out);

  const fs::path ffn_dir = dir / "ffn";
  fs::create_directories(ffn_dir, ec);
  if (ec) throw InvalidOperationException("Could not create '" + ffn_dir.string() + "': " + ec.message());
  for (size_t i = 0; i < Blocks.size(); ++i)
    write_file(ffn_dir / ("ffn_layer_" + std::to_string(i) + ".json"), ffn_json(Blocks[i].FeedForward, c));
}

LanguageModel LanguageModel::Load(const std::string &directory, HipAccelerationManager *accel) {
  const fs::path dir(directory);
  const auto vals = read_config_values(dir / "config.json");
  auto get = [&](const char *k) -> const ConfigValue & {
    auto it = vals.find(k);
    if (it == vals.end())
      throw InvalidOperationException("config.json: the given key '" + std::string(k) + "' was not present.");
    return it->second;
  };
  // JsonElement.GetInt32 / GetBoolean / GetSingle
  auto get_int = [&](const char *k) {
    const ConfigValue &v = get(k);
    char *end = nullptr;
    const long long x = v.kind == ConfigValue::Number ? std::strtoll(v.text.c_str(), &end, 10) : 0;
    if (v.kind != ConfigValue::Number || *end || x < INT32_MIN || x > INT32_MAX)
      throw InvalidOperationException("config.json: '" + std::string(k) + "' is not a 32-bit integer.");
    return (int)x;
  };
  auto get_bool = [&](const char *k) {
    const ConfigValue &v = get(k);
    if (v.kind != ConfigValue::Bool)
      throw InvalidOperationException("config.json: '" + std::string(k) + "' is not true or false.");
    return v.flag;
  };
  auto get_float = [&](const char *k) {
    const ConfigValue &v = get(k);
    char *end = nullptr;
    const float x = v.kind == ConfigValue::Number ? std::strtof(v.text.c_str(), &end) : 0.f;
    if (v.kind != ConfigValue::Number || *end)
      throw InvalidOperationException("config.json: '" + std::string(k) + "' is not a number.");
    return x;
  };
  TransformerConfig c;
  c.VocabSize = get_int("VocabSize");
  c.MaxSequenceLength = get_int("MaxSequenceLength");
  c.EmbeddingDim = get_int("EmbeddingDim");
  c.NumHeads = get_int("NumHeads");
  c.NumLayers = get_int("NumLayers");
  c.FeedForwardDim = get_int("FeedForwardDim");
  c.UseDecoderOnly = get_bool("UseDecoderOnly");
  c.InputFeatureDim = get_int("InputFeatureDim");
  c.OutputDim = get_int("OutputDim");
  c.FFNActivationType = get_int("FFNActivationType");
  c.AccelerationType = get_int("AccelerationType");
  c.AccelerationDeviceId = get_int("AccelerationDeviceId");
  c.L2RegulationLamda = get_float("L2RegulationLamda");
  c.GradientClippingThreshold = get_float("GradientClippingThreshold");
  c.DataType = get_int("DataType");
  c.CostFunction = get_int("CostFunction");
  c.ActivationDistribution = get_int("ActivationDistribution");
  c.UsesDiscreteTokens = c.DataType == 0 || c.DataType == 3;  // DataConfig.cs:23-25
  c.Validate();

  LanguageModel model(c, accel);
  const fs::path wpath = dir / "weights.bin";
  const std::string bytes = read_file(wpath);
  BinReader r(bytes, wpath.string());
  const bool saved_discrete = r.boolean();
  // ReadMatrixInto on the member the config did not create (null in the
  // reference) throws ArgumentNullException("m").
  if (saved_discrete != c.UsesDiscreteTokens) throw ArgumentNullException("m");
  if (saved_discrete) {
    r.matrix_into(model.TokenEmbedding);
  } else {
    r.matrix_into(model.InputProjection);
    r.vector_into(model.InputProjectionBias);
  }
  for (TransformerBlock &b : model.Blocks) {
    MultiHeadAttention &a = b.Attention;
    r.matrix_into(a.WQ);
    r.matrix_into(a.WK);
    r.matrix_into(a.WV);
    r.matrix_into(a.WO);
    r.vector_into(a.BiasQ);
    r.vector_into(a.BiasK);
    r.vector_into(a.BiasV);
    r.vector_into(a.BiasO);
    r.vector_into(b.LN1Gamma);
    r.vector_into(b.LN1Beta);
    r.vector_into(b.LN2Gamma);
    r.vector_into(b.LN2Beta);
  }
  r.matrix_into(model.OutputProjection);
  r.vector_into(model.OutputBias);

  for (size_t i = 0; i < model.Blocks.size(); ++i) {
    const fs::path p = dir / "ffn" / ("ffn_layer_" + std::to_string(i) + ".json");
    if (!fs::exists(p)) throw FileNotFoundException("Missing FFN file: " + p.string());
    model.Blocks[i].FeedForward = read_ffn(p);
  }
  return model;
}

}  // namespace cdml_host

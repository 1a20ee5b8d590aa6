// Python module _cdml_host: the C++ host side (HipAccelerationManager and the
// MultiTypeTransformer classes) on numpy arrays, for the parity tests, the
// smoke check and the benchmark.  float32 arrays are passed by pointer; the
// manager's resident cache keys weights by those pointers exactly as the C#
// manager keys them by array identity.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <chrono>
#include <cstring>

#include "cdml_host.h"

namespace py = pybind11;
using namespace cdml_host;

namespace {

using F32 = py::array_t<float, py::array::c_style | py::array::forcecast>;
using I32 = py::array_t<int, py::array::c_style | py::array::forcecast>;
using U8 = py::array_t<uint8_t, py::array::c_style | py::array::forcecast>;

// Arrays handed to the C++ side stay alive for the duration of the call
// through these holders.
struct MatArg {
  F32 arr;
  MatView view;
};

MatArg mat(const py::object &o) {
  MatArg a;
  if (o.is_none()) return a;
  a.arr = F32::ensure(o);
  if (!a.arr) throw ArgumentException("expected a float32 matrix");
  if (a.arr.ndim() != 2) throw ArgumentException("expected a 2-D array");
  a.view = MatView(a.arr.data(), (int)a.arr.shape(0), (int)a.arr.shape(1));
  return a;
}

struct VecArg {
  F32 arr;
  VecView view;
};

VecArg vec(const py::object &o) {
  VecArg a;
  if (o.is_none()) return a;
  a.arr = F32::ensure(o);
  if (!a.arr) throw ArgumentException("expected a float32 vector");
  if (a.arr.ndim() != 1) throw ArgumentException("expected a 1-D array");
  a.view = VecView(a.arr.data(), (int)a.arr.shape(0));
  return a;
}

struct MaskArg {
  U8 arr;
  MaskView view;
};

MaskArg mask(const py::object &o) {
  MaskArg a;
  if (o.is_none()) return a;
  a.arr = U8::ensure(o);
  if (!a.arr || a.arr.ndim() != 2) throw ArgumentException("expected a 2-D bool mask", "mask");
  a.view.data = a.arr.data();
  a.view.rows = (int)a.arr.shape(0);
  a.view.cols = (int)a.arr.shape(1);
  return a;
}

// In-place arguments must be writable float32 C-contiguous arrays (no copy).
MatRef mat_inplace(py::array &a) {
  if (!(a.flags() & py::array::c_style) || !a.dtype().is(py::dtype::of<float>()) || a.ndim() != 2 ||
      !a.writeable())
    throw ArgumentException("in-place argument must be a writable float32 C-contiguous matrix");
  return MatRef(static_cast<float *>(a.mutable_data()), (int)a.shape(0), (int)a.shape(1));
}

// Gradient accumulators: writable float32 C-contiguous arrays, None = null.
MatRef mat_inout(const py::object &o) {
  if (o.is_none()) return MatRef();
  py::array a = o;
  return mat_inplace(a);
}

VecRef vec_inout(const py::object &o) {
  if (o.is_none()) return VecRef();
  py::array a = o;
  if (!(a.flags() & py::array::c_style) || !a.dtype().is(py::dtype::of<float>()) || a.ndim() != 1 ||
      !a.writeable())
    throw ArgumentException("in-place argument must be a writable float32 C-contiguous vector");
  return VecRef(static_cast<float *>(a.mutable_data()), (int)a.shape(0));
}

py::array_t<float> to_numpy(Matrix &&m) {
  auto *v = new FloatBuf(std::move(m.data));
  py::capsule owner(v, [](void *p) { delete static_cast<FloatBuf *>(p); });
  return py::array_t<float>({(py::ssize_t)m.rows, (py::ssize_t)m.cols},
                            {(py::ssize_t)(m.cols * sizeof(float)), (py::ssize_t)sizeof(float)}, v->data(),
                            owner);
}

py::array_t<float> to_numpy(const Matrix &m) { return to_numpy(Matrix(m)); }

py::array_t<float> vec_to_numpy(const std::vector<float> &v) {
  py::array_t<float> a((py::ssize_t)v.size());
  if (!v.empty()) std::memcpy(a.mutable_data(), v.data(), v.size() * sizeof(float));
  return a;
}

Matrix from_numpy(const py::object &o) {
  MatArg a = mat(o);
  if (a.view.null()) throw ArgumentNullException("matrix");
  Matrix m(a.view.rows, a.view.cols);
  std::memcpy(m.ptr(), a.view.data, m.data.size() * sizeof(float));
  return m;
}

std::vector<float> vec_from_numpy(const py::object &o) {
  VecArg a = vec(o);
  if (a.view.null()) throw ArgumentNullException("vector");
  return std::vector<float>(a.view.data, a.view.data + a.view.length);
}

// Weights in the layout of cdml.synth.lm_weights.
void load_weights(LanguageModel &lm, const py::dict &w) {
  auto get = [&](const py::dict &d, const char *k) -> py::object {
    if (!d.contains(k)) throw ArgumentException(std::string("missing weight '") + k + "'");
    return d[k];
  };
  auto assign_mat = [](Matrix &dst, const py::object &o, const char *name) {
    Matrix m = from_numpy(o);
    if (m.rows != dst.rows || m.cols != dst.cols)
      throw ArgumentException(std::string("shape mismatch for ") + name);
    dst = std::move(m);
  };
  auto assign_vec = [](std::vector<float> &dst, const py::object &o, const char *name) {
    std::vector<float> v = vec_from_numpy(o);
    if (v.size() != dst.size()) throw ArgumentException(std::string("length mismatch for ") + name);
    dst = std::move(v);
  };
  const TransformerConfig &c = lm.config();
  if (c.UsesDiscreteTokens) {
    assign_mat(lm.TokenEmbedding, get(w, "token_embedding"), "token_embedding");
  } else {
    assign_mat(lm.InputProjection, get(w, "input_proj"), "input_proj");
    assign_vec(lm.InputProjectionBias, get(w, "input_bias"), "input_bias");
  }
  assign_mat(lm.OutputProjection, get(w, "out_proj"), "out_proj");
  assign_vec(lm.OutputBias, get(w, "out_bias"), "out_bias");
  py::list layers = get(w, "layers");
  if ((int)py::len(layers) != c.NumLayers) throw ArgumentException("layer count mismatch");
  for (int i = 0; i < c.NumLayers; ++i) {
    py::dict L = layers[i];
    TransformerBlock &b = lm.Blocks[i];
    assign_mat(b.Attention.WQ, get(L, "wq"), "wq");
    assign_mat(b.Attention.WK, get(L, "wk"), "wk");
    assign_mat(b.Attention.WV, get(L, "wv"), "wv");
    assign_mat(b.Attention.WO, get(L, "wo"), "wo");
    assign_vec(b.Attention.BiasQ, get(L, "bq"), "bq");
    assign_vec(b.Attention.BiasK, get(L, "bk"), "bk");
    assign_vec(b.Attention.BiasV, get(L, "bv"), "bv");
    assign_vec(b.Attention.BiasO, get(L, "bo"), "bo");
    assign_vec(b.LN1Gamma, get(L, "ln1_g"), "ln1_g");
    assign_vec(b.LN1Beta, get(L, "ln1_b"), "ln1_b");
    assign_vec(b.LN2Gamma, get(L, "ln2_g"), "ln2_g");
    assign_vec(b.LN2Beta, get(L, "ln2_b"), "ln2_b");
    assign_mat(b.FeedForward.weights[0], get(L, "ffn_w1"), "ffn_w1");
    assign_vec(b.FeedForward.biases[0], get(L, "ffn_b1"), "ffn_b1");
    assign_mat(b.FeedForward.weights[1], get(L, "ffn_w2"), "ffn_w2");
    assign_vec(b.FeedForward.biases[1], get(L, "ffn_b2"), "ffn_b2");
  }
}

std::vector<int> ids_from(const py::object &o) {
  I32 a = I32::ensure(o);
  if (!a) throw ArgumentNullException("tokenIds");
  return std::vector<int>(a.data(), a.data() + a.size());
}

// Runs f with the GIL released: the manager's methods only touch C++ data
// and the numpy buffers that the argument holders keep alive, so other
// Python threads (other managers) run meanwhile.
template <class F>
auto nogil(F &&f) -> decltype(f()) {
  py::gil_scoped_release release;
  return f();
}

}  // namespace

PYBIND11_MODULE(_cdml_host, m) {
  m.doc() = "C++ host side of the gfx950 attention path (HipAccelerationManager and models)";

  auto arg_exc = py::register_exception<ArgumentException>(m, "ArgumentException", PyExc_ValueError);
  py::register_exception<ArgumentNullException>(m, "ArgumentNullException", arg_exc.ptr());
  py::register_exception<ArgumentOutOfRangeException>(m, "ArgumentOutOfRangeException", arg_exc.ptr());
  py::register_exception<InvalidOperationException>(m, "InvalidOperationException", PyExc_RuntimeError);
  py::register_exception<FileNotFoundException>(m, "FileNotFoundException", PyExc_FileNotFoundError);

  m.def("sdpa_backward_workspace_choice",
        // the drop-in attention backward's workspace size for one sequence
        // (MultiHeadAttentionBackward): the C ABI's two sizes and the choice
        [](int lq, int lk, int dim, int numHeads, bool causal, size_t extra_cap) {
          size_t base = 0, stored = 0;
          if (cdml_sdpa_bwd_workspace_size(1, lq, lk, dim, numHeads, &base) != CDML_OK ||
              cdml_sdpa_bwd_stored_ds_workspace_size(1, lq, lk, dim, numHeads, causal ? 1 : 0, &stored) != CDML_OK)
            throw ArgumentException(cdml_last_error());
          return py::make_tuple(base, stored, SdpaBackwardWorkspaceChoice(base, stored, extra_cap));
        },
        py::arg("lq"), py::arg("lk"), py::arg("dim"), py::arg("numHeads"), py::arg("causal"),
        py::arg("extra_cap") = kStoredDsExtraBytesCap);
  m.attr("STORED_DS_EXTRA_BYTES_CAP") = kStoredDsExtraBytesCap;

  py::class_<HipAccelerationManager>(m, "HipAccelerationManager")
      .def(py::init<int>(), py::arg("device") = 0)
      .def("ProjectQKV",
           [](HipAccelerationManager &a, py::object x, py::object wq, py::object bq, py::object wk,
              py::object bk, py::object wv, py::object bv) {
             auto X = mat(x), WQ = mat(wq), WK = mat(wk), WV = mat(wv);
             auto BQ = vec(bq), BK = vec(bk), BV = vec(bv);
             auto r = nogil([&] { return a.ProjectQKV(X.view, WQ.view, BQ.view, WK.view, BK.view, WV.view, BV.view); });
             return py::make_tuple(to_numpy(std::move(std::get<0>(r))), to_numpy(std::move(std::get<1>(r))),
                                   to_numpy(std::move(std::get<2>(r))));
           })
      .def("ScaledDotProductAttention",
           [](HipAccelerationManager &a, py::object q, py::object k, py::object v, int numHeads,
              py::object msk, bool causal) {
             auto Q = mat(q), K = mat(k), V = mat(v);
             auto M = mask(msk);
             return to_numpy(nogil([&] { return a.ScaledDotProductAttention(Q.view, K.view, V.view, numHeads, M.view, causal); }));
           },
           py::arg("q"), py::arg("k"), py::arg("v"), py::arg("numHeads"), py::arg("mask") = py::none(),
           py::arg("causal") = false)
      .def("MultiHeadAttentionForward",
           [](HipAccelerationManager &a, py::object q, py::object k, py::object v, int numHeads,
              float scale, py::object msk) {
             auto Q = mat(q), K = mat(k), V = mat(v);
             auto M = mask(msk);
             return to_numpy(nogil([&] { return a.MultiHeadAttentionForward(Q.view, K.view, V.view, numHeads, scale, M.view); }));
           },
           py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("numHeads"), py::arg("scale"),
           py::arg("mask") = py::none())
      .def("ProjectOutputBatch",
           [](HipAccelerationManager &a, py::object h, py::object w, py::object b, int seqLen, int outputDim) {
             auto Hh = mat(h), W = mat(w);
             auto B = vec(b);
             return to_numpy(nogil([&] { return a.ProjectOutputBatch(Hh.view, W.view, B.view, seqLen, outputDim); }));
           })
      .def("BatchDotProductAddBias",
           [](HipAccelerationManager &a, py::object w, py::object x, py::object b) {
             auto W = mat(w), X = mat(x);
             auto B = vec(b);
             return to_numpy(nogil([&] { return a.BatchDotProductAddBias(W.view, X.view, B.view); }));
           })
      .def("BatchDotProductAddBias",
           [](HipAccelerationManager &a, py::object w, py::object x, int rowStart, int rowCount, py::object b) {
             auto W = mat(w), X = mat(x);
             auto B = vec(b);
             return to_numpy(nogil([&] { return a.BatchDotProductAddBias(W.view, X.view, rowStart, rowCount, B.view); }));
           })
      .def("ApplyRotaryPositionEmbeddingInPlace",
           [](HipAccelerationManager &a, py::object mtx, int numHeads, float baseTheta, bool inverse) {
             if (mtx.is_none()) throw ArgumentNullException("matrix");
             py::array arr = mtx;
             MatRef m = mat_inplace(arr);
             nogil([&] { a.ApplyRotaryPositionEmbeddingInPlace(m, numHeads, baseTheta, inverse); });
           })
      .def("ApplyRotaryPositionEmbeddingHeadInPlace",
           [](HipAccelerationManager &a, py::object mtx, int startCol, int headDim, float baseTheta,
              bool inverse) {
             if (mtx.is_none()) throw ArgumentNullException("matrix");
             py::array arr = mtx;
             MatRef m = mat_inplace(arr);
             nogil([&] { a.ApplyRotaryPositionEmbeddingHeadInPlace(m, startCol, headDim, baseTheta, inverse); });
           })
      .def("ResidualLayerNorm",
           [](HipAccelerationManager &a, py::object x, py::object s, py::object g, py::object b, float eps) {
             auto X = mat(x), S = mat(s);
             auto G = vec(g), B = vec(b);
             return to_numpy(nogil([&] { return a.ResidualLayerNorm(X.view, S.view, G.view, B.view, eps); }));
           },
           py::arg("input"), py::arg("subLayer"), py::arg("gamma"), py::arg("beta"), py::arg("epsilon") = 1e-5f)
      .def("EmbedTokenIds",
           [](HipAccelerationManager &a, py::object ids, py::object emb, int dim) {
             if (ids.is_none()) throw ArgumentNullException("tokenIds");
             auto E = mat(emb);
             std::vector<int> I = ids_from(ids);
             return to_numpy(nogil([&] { return a.EmbedTokenIds(I, E.view, dim); }));
           })
      .def("EmbedTokenIds",
           [](HipAccelerationManager &a, py::object ids, int start, int count, py::object emb, int dim) {
             if (ids.is_none()) throw ArgumentNullException("tokenIds");
             auto E = mat(emb);
             std::vector<int> I = ids_from(ids);
             return to_numpy(nogil([&] { return a.EmbedTokenIds(I, start, count, E.view, dim); }));
           })
      .def("CreateCausalMask",
           [](HipAccelerationManager &a, int n) {
             BoolMatrix b = a.CreateCausalMask(n);
             py::array_t<bool> out({(py::ssize_t)b.rows, (py::ssize_t)b.cols});
             std::memcpy(out.mutable_data(), b.data.data(), b.data.size());
             return out;
           })
      .def("FFNForwardBatch",
           [](HipAccelerationManager &a, py::object x, int seqLen, int outputDim, py::list ws, py::list bs,
              std::vector<int> acts) {
             auto X = mat(x);
             FeedForwardNetwork ffn;
             for (auto w : ws) ffn.weights.push_back(from_numpy(py::reinterpret_borrow<py::object>(w)));
             for (auto b : bs) ffn.biases.push_back(vec_from_numpy(py::reinterpret_borrow<py::object>(b)));
             ffn.activations = acts;
             if (ffn.biases.size() != ffn.weights.size() || ffn.activations.size() != ffn.weights.size())
               throw ArgumentException("FFN weights, biases and activations must have equal counts");
             return to_numpy(nogil([&] { return a.FFNForwardBatch(X.view, seqLen, outputDim, ffn); }));
           })
      .def("DecodeSelfAttention",
           [](HipAccelerationManager &a, py::array q, py::array k, py::object v, py::array keys,
              py::array values, int pos, int numHeads) {
             auto V = mat(v);
             MatRef Q = mat_inplace(q), K = mat_inplace(k), KS = mat_inplace(keys), VS = mat_inplace(values);
             return to_numpy(nogil([&] { return a.DecodeSelfAttention(Q, K, V.view, KS, VS, pos, numHeads); }));
           })
      .def("MultiHeadAttentionBackward",
           [](HipAccelerationManager &a, py::object q, py::object k, py::object v, py::object dout,
              int numHeads, float scale, py::object maskOrDecoder) {
             auto Q = mat(q), K = mat(k), V = mat(v), D = mat(dout);
             std::tuple<Matrix, Matrix, Matrix> r;
             if (py::isinstance<py::bool_>(maskOrDecoder)) {  // the useDecoderMask overload
               const bool dec = maskOrDecoder.cast<bool>();
               r = nogil([&] { return a.MultiHeadAttentionBackward(Q.view, K.view, V.view, D.view, numHeads, scale, dec); });
             }
             else {
               auto M = mask(maskOrDecoder);
               r = nogil([&] { return a.MultiHeadAttentionBackward(Q.view, K.view, V.view, D.view, numHeads, scale, M.view); });
             }
             return py::make_tuple(to_numpy(std::move(std::get<0>(r))), to_numpy(std::move(std::get<1>(r))),
                                   to_numpy(std::move(std::get<2>(r))));
           },
           py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("dConcatenated"), py::arg("numHeads"),
           py::arg("scale"), py::arg("mask") = false)
      .def("BackpropQKV",
           [](HipAccelerationManager &a, py::object x, py::object dq, py::object dk, py::object dv,
              py::object wq, py::object wk, py::object wv, py::object wqg, py::object bqg, py::object wkg,
              py::object bkg, py::object wvg, py::object bvg) {
             auto X = mat(x), DQ = mat(dq), DK = mat(dk), DV = mat(dv), WQ = mat(wq), WK = mat(wk),
                  WV = mat(wv);
             MatRef GQ = mat_inout(wqg), GK = mat_inout(wkg), GV = mat_inout(wvg);
             VecRef BQ = vec_inout(bqg), BK = vec_inout(bkg), BV = vec_inout(bvg);
             return to_numpy(nogil([&] {
               return a.BackpropQKV(X.view, DQ.view, DK.view, DV.view, WQ.view, WK.view, WV.view, GQ, BQ, GK, BK, GV, BV);
             }));
           })
      .def("BackpropLinearProjection",
           [](HipAccelerationManager &a, py::object x, py::object dy, py::object w, py::object wg,
              py::object bg, py::object dx) {
             auto X = mat(x), DY = mat(dy), W = mat(w);
             MatRef WG = mat_inout(wg), DX = mat_inout(dx);
             VecRef BG = vec_inout(bg);
             nogil([&] { a.BackpropLinearProjection(X.view, DY.view, W.view, WG, BG, DX); });
           })
      .def("BackpropOutputProjection",
           [](HipAccelerationManager &a, py::object dl, py::object x, py::object w, py::object wg,
              py::object bg, int seqLen, int outputDim, int embeddingDim) {
             auto DL = mat(dl), X = mat(x), W = mat(w);
             MatRef WG = mat_inout(wg);
             VecRef BG = vec_inout(bg);
             return to_numpy(nogil([&] {
               return a.BackpropOutputProjection(DL.view, X.view, W.view, WG, BG, seqLen, outputDim, embeddingDim);
             }));
           })
      .def("BackpropInputProjection",
           [](HipAccelerationManager &a, py::object dx, py::object x, int rowStart, py::object wg, py::object bg,
              int seqLen, int embeddingDim, int inputFeatureDim) {
             auto DX = mat(dx), X = mat(x);
             MatRef WG = mat_inout(wg);
             VecRef BG = vec_inout(bg);
             nogil([&] {
               a.BackpropInputProjection(DX.view, X.view, rowStart, WG, BG, seqLen, embeddingDim, inputFeatureDim);
               return 0;
             });
           })
      .def("MatrixMultiply",
           [](HipAccelerationManager &a, py::object A, py::object B) {
             auto X = mat(A), Y = mat(B);
             return to_numpy(nogil([&] { return a.MatrixMultiply(X.view, Y.view); }));
           })
      .def("MatrixMultiplyTranspose",
           [](HipAccelerationManager &a, py::object A, py::object B) {
             auto X = mat(A), Y = mat(B);
             return to_numpy(nogil([&] { return a.MatrixMultiplyTranspose(X.view, Y.view); }));
           })
      .def("ResidualLayerNormForward",
           [](HipAccelerationManager &a, py::object x, py::object sl, py::object g, py::object b, float eps) {
             auto X = mat(x), S = mat(sl);
             auto G = vec(g), B = vec(b);
             auto r = nogil([&] { return a.ResidualLayerNormForward(X.view, S.view, G.view, B.view, eps); });
             return py::make_tuple(to_numpy(std::move(std::get<0>(r))), vec_to_numpy(std::get<1>(r)),
                                   vec_to_numpy(std::get<2>(r)), to_numpy(std::move(std::get<3>(r))),
                                   to_numpy(std::move(std::get<4>(r))));
           },
           py::arg("input"), py::arg("subLayer"), py::arg("gamma"), py::arg("beta"), py::arg("epsilon") = 1e-5f)
      .def("LayerNormBackward",
           [](HipAccelerationManager &a, py::object d, py::object n, py::object g, py::object x, py::object m,
              py::object v, float eps) {
             auto D = mat(d), Nn = mat(n), X = mat(x);
             auto G = vec(g), M = vec(m), V = vec(v);
             auto r = nogil([&] { return a.LayerNormBackward(D.view, Nn.view, G.view, X.view, M.view, V.view, eps); });
             return py::make_tuple(to_numpy(std::move(std::get<0>(r))), vec_to_numpy(std::get<1>(r)),
                                   vec_to_numpy(std::get<2>(r)));
           },
           py::arg("dOut"), py::arg("normalized"), py::arg("gamma"), py::arg("input"), py::arg("mean"),
           py::arg("variance"), py::arg("epsilon") = 1e-5f)
      .def("CrossEntropyLossAndGradient",
           [](HipAccelerationManager &a, py::object logits, py::object targets, int targetStart, int effectiveLen) {
             if (targets.is_none()) throw ArgumentNullException("targets");
             auto L = mat(logits);
             std::vector<int> T = ids_from(targets);
             auto r = nogil([&] { return a.CrossEntropyLossAndGradient(L.view, T, targetStart, effectiveLen); });
             return py::make_tuple(r.first, to_numpy(std::move(r.second)));
           },
           py::arg("logits"), py::arg("targets"), py::arg("targetStart"), py::arg("effectiveLen"))
      .def("MSELossAndGradient",
           [](HipAccelerationManager &a, py::object pred, py::object targets, int targetStart, int effectiveLen) {
             auto P = mat(pred);
             auto T = mat(targets);
             auto r = nogil([&] { return a.MSELossAndGradient(P.view, T.view, targetStart, effectiveLen); });
             return py::make_tuple(r.first, to_numpy(std::move(r.second)));
           },
           py::arg("predictions"), py::arg("targets"), py::arg("targetStart"), py::arg("effectiveLen"))
      .def("AccumulateTokenEmbeddingGrad",
           [](HipAccelerationManager &a, py::object eg, py::object dx, py::object ids, int tokenStart, int seqLen,
              int dim) {
             if (ids.is_none()) throw ArgumentNullException("tokenIds");
             auto D = mat(dx);
             MatRef EG = mat_inout(eg);
             std::vector<int> I = ids_from(ids);
             nogil([&] { a.AccumulateTokenEmbeddingGrad(EG, D.view, I, tokenStart, seqLen, dim); });
           })
      .def("ZeroMatrix",
           [](HipAccelerationManager &a, py::object m) {
             if (m.is_none()) throw ArgumentNullException("matrix");
             MatRef M = mat_inout(m);
             nogil([&] { a.ZeroMatrix(M); });
           })
      .def("ZeroVector",
           [](HipAccelerationManager &a, py::object v) {
             if (v.is_none()) throw ArgumentNullException("vector");
             VecRef Vv = vec_inout(v);
             nogil([&] { a.ZeroVector(Vv); });
           })
      .def("MatrixAddInPlace",
           [](HipAccelerationManager &a, py::object t, py::object x) {
             MatRef T = mat_inout(t);
             auto X = mat(x);
             nogil([&] { a.MatrixAddInPlace(T, X.view); });
           })
      .def("VectorAccumulate",
           [](HipAccelerationManager &a, py::object t, py::object x) {
             VecRef T = vec_inout(t);
             auto X = vec(x);
             nogil([&] { a.VectorAccumulate(T, X.view); });
           })
      .def("MatrixSquaredNorm",
           [](HipAccelerationManager &a, py::object m) {
             auto M = mat(m);
             return nogil([&] { return a.MatrixSquaredNorm(M.view); });
           })
      .def("VectorSquaredNorm",
           [](HipAccelerationManager &a, py::object v) {
             auto Vv = vec(v);
             return nogil([&] { return a.VectorSquaredNorm(Vv.view); });
           })
      .def("MatrixScaleInPlace",
           [](HipAccelerationManager &a, py::object m, float scale) {
             MatRef M = mat_inout(m);
             nogil([&] { a.MatrixScaleInPlace(M, scale); });
           })
      .def("VectorScaleInPlace",
           [](HipAccelerationManager &a, py::object v, float scale) {
             VecRef Vv = vec_inout(v);
             nogil([&] { a.VectorScaleInPlace(Vv, scale); });
           })
      .def("MatrixUpdate",
           [](HipAccelerationManager &a, py::object w, py::object g, float lr) {
             MatRef W = mat_inout(w);
             auto G = mat(g);
             nogil([&] { a.MatrixUpdate(W, G.view, lr); });
           })
      .def("VectorUpdate",
           [](HipAccelerationManager &a, py::object w, py::object g, float lr) {
             VecRef W = vec_inout(w);
             auto G = vec(g);
             nogil([&] { a.VectorUpdate(W, G.view, lr); });
           })
      .def("SegmentedAttentionForward",
           [](HipAccelerationManager &a, py::object q, py::object k, py::object v, int numHeads, int segLen,
              int segCount, bool causal) {
             auto Q = mat(q), K = mat(k), V = mat(v);
             return to_numpy(nogil([&] {
               return a.SegmentedAttentionForward(Q.view, K.view, V.view, numHeads, segLen, segCount, causal);
             }));
           })
      .def("SegmentedMultiHeadAttentionBackward",
           [](HipAccelerationManager &a, py::object q, py::object k, py::object v, py::object d, int numHeads,
              float scale, int segLen, int segCount, bool causal) {
             auto Q = mat(q), K = mat(k), V = mat(v), Dd = mat(d);
             auto r = nogil([&] {
               return a.SegmentedMultiHeadAttentionBackward(Q.view, K.view, V.view, Dd.view, numHeads, scale, segLen,
                                                            segCount, causal);
             });
             return py::make_tuple(to_numpy(std::move(std::get<0>(r))), to_numpy(std::move(std::get<1>(r))),
                                   to_numpy(std::move(std::get<2>(r))));
           })
      .def("ApplySegmentedRotaryInPlace",
           [](HipAccelerationManager &a, py::object q, py::object k, int numHeads, int segLen, bool inverse) {
             MatRef Q = mat_inout(q), K = mat_inout(k);
             if (!Q.data || !K.data) throw ArgumentNullException(!Q.data ? "q" : "k");
             nogil([&] { a.ApplySegmentedRotaryInPlace(Q, K, numHeads, segLen, inverse); });
           })
      .def("FFNInputGradientBatch",
           [](HipAccelerationManager &a, py::object x, py::object dy, py::list ws, py::list bs, std::vector<int> acts,
              py::list wgs, py::list bgs) {
             auto X = mat(x), DY = mat(dy);
             FeedForwardNetwork ffn;
             for (auto w : ws) ffn.weights.push_back(from_numpy(py::reinterpret_borrow<py::object>(w)));
             for (auto b : bs) ffn.biases.push_back(vec_from_numpy(py::reinterpret_borrow<py::object>(b)));
             ffn.activations = acts;
             if (ffn.biases.size() != ffn.weights.size() || ffn.activations.size() != ffn.weights.size())
               throw ArgumentException("FFN weights, biases and activations must have equal counts");
             std::vector<MatRef> WG;
             std::vector<VecRef> BG;
             for (auto w : wgs) WG.push_back(mat_inout(py::reinterpret_borrow<py::object>(w)));
             for (auto b : bgs) BG.push_back(vec_inout(py::reinterpret_borrow<py::object>(b)));
             return to_numpy(nogil([&] { return a.FFNInputGradientBatch(X.view, DY.view, ffn, WG, BG); }));
           })
      .def("SetActivationCacheLimit", &HipAccelerationManager::SetActivationCacheLimit, py::arg("bytes"))
      .def_property_readonly("activation_cache_limit", &HipAccelerationManager::activation_cache_limit)
      .def_property_readonly("activation_cache_entries", &HipAccelerationManager::activation_cache_entries)
      .def("transfer_stats",
           [](HipAccelerationManager &a) {
             auto t = a.transfer_stats();
             py::dict d;
             d["h2d_bytes"] = t.h2d_bytes;
             d["d2h_bytes"] = t.d2h_bytes;
             d["h2d_skipped_bytes"] = t.h2d_skipped_bytes;
             d["backward_from_saved"] = t.backward_from_saved;
             d["act_alloc_failures"] = t.act_alloc_failures;
             return d;
           })
      .def_static("SetProcessActivationCacheBudget", &HipAccelerationManager::SetProcessActivationCacheBudget)
      .def_static("ProcessActivationCacheBudget", &HipAccelerationManager::ProcessActivationCacheBudget)
      .def_static("ProcessActivationCacheBytes", &HipAccelerationManager::ProcessActivationCacheBytes)
      .def_static("InjectActivationAllocFailures", &HipAccelerationManager::InjectActivationAllocFailures)
      .def("Dispose", &HipAccelerationManager::Dispose);
  m.def("host_copy_threads", &HostCopyThreads);
  // The host copy engine on byte arrays (for tests of its slicing).
  m.def("_parallel_copy", [](py::array_t<uint8_t, py::array::c_style | py::array::forcecast> a) {
    py::array_t<uint8_t> out(a.size());
    ParallelMemcpy(out.mutable_data(), a.data(), (size_t)a.size());
    return out;
  });
  m.def("_parallel_equal", [](py::array_t<uint8_t, py::array::c_style | py::array::forcecast> a,
                              py::array_t<uint8_t, py::array::c_style | py::array::forcecast> b) {
    if (a.size() != b.size()) return false;
    return ParallelEqual(a.data(), b.data(), (size_t)a.size());
  });

  py::class_<TransformerConfig>(m, "TransformerConfig")
      .def(py::init<>())
      .def_readwrite("VocabSize", &TransformerConfig::VocabSize)
      .def_readwrite("MaxSequenceLength", &TransformerConfig::MaxSequenceLength)
      .def_readwrite("EmbeddingDim", &TransformerConfig::EmbeddingDim)
      .def_readwrite("NumHeads", &TransformerConfig::NumHeads)
      .def_readwrite("NumLayers", &TransformerConfig::NumLayers)
      .def_readwrite("FeedForwardDim", &TransformerConfig::FeedForwardDim)
      .def_readwrite("UseDecoderOnly", &TransformerConfig::UseDecoderOnly)
      .def_readwrite("UsesDiscreteTokens", &TransformerConfig::UsesDiscreteTokens)
      .def_readwrite("InputFeatureDim", &TransformerConfig::InputFeatureDim)
      .def_readwrite("OutputDim", &TransformerConfig::OutputDim)
      .def_readwrite("FFNActivationType", &TransformerConfig::FFNActivationType)
      .def_readwrite("DataType", &TransformerConfig::DataType)
      .def_readwrite("AccelerationType", &TransformerConfig::AccelerationType)
      .def_readwrite("AccelerationDeviceId", &TransformerConfig::AccelerationDeviceId)
      .def_readwrite("L2RegulationLamda", &TransformerConfig::L2RegulationLamda)
      .def_readwrite("GradientClippingThreshold", &TransformerConfig::GradientClippingThreshold)
      .def_readwrite("CostFunction", &TransformerConfig::CostFunction)
      .def_readwrite("ActivationDistribution", &TransformerConfig::ActivationDistribution)
      .def("Validate", &TransformerConfig::Validate);

  py::class_<LanguageModel>(m, "LanguageModel")
      .def(py::init<const TransformerConfig &, HipAccelerationManager *>(), py::keep_alive<1, 3>())
      .def("load_weights", &load_weights)
      .def("Save", &LanguageModel::Save, py::arg("directory"))
      .def_static("Load", &LanguageModel::Load, py::arg("directory"), py::arg("accel"), py::keep_alive<0, 2>())
      .def_property_readonly("config", &LanguageModel::config)
      .def("weights",
           [](const LanguageModel &lm) {
             // the cdml.synth.lm_weights layout (arrays copied out)
             py::dict w;
             const TransformerConfig &c = lm.config();
             if (c.UsesDiscreteTokens) {
               w["token_embedding"] = to_numpy(lm.TokenEmbedding);
             } else {
               w["input_proj"] = to_numpy(lm.InputProjection);
               w["input_bias"] = vec_to_numpy(lm.InputProjectionBias);
             }
             w["out_proj"] = to_numpy(lm.OutputProjection);
             w["out_bias"] = vec_to_numpy(lm.OutputBias);
             py::list layers;
             for (const TransformerBlock &b : lm.Blocks) {
               py::dict L;
               L["wq"] = to_numpy(b.Attention.WQ);
               L["wk"] = to_numpy(b.Attention.WK);
               L["wv"] = to_numpy(b.Attention.WV);
               L["wo"] = to_numpy(b.Attention.WO);
               L["bq"] = vec_to_numpy(b.Attention.BiasQ);
               L["bk"] = vec_to_numpy(b.Attention.BiasK);
               L["bv"] = vec_to_numpy(b.Attention.BiasV);
               L["bo"] = vec_to_numpy(b.Attention.BiasO);
               L["ln1_g"] = vec_to_numpy(b.LN1Gamma);
               L["ln1_b"] = vec_to_numpy(b.LN1Beta);
               L["ln2_g"] = vec_to_numpy(b.LN2Gamma);
               L["ln2_b"] = vec_to_numpy(b.LN2Beta);
               py::list fw, fb, fa;
               for (size_t i = 0; i < b.FeedForward.weights.size(); ++i) {
                 fw.append(to_numpy(b.FeedForward.weights[i]));
                 fb.append(vec_to_numpy(b.FeedForward.biases[i]));
                 fa.append(b.FeedForward.activations[i]);
               }
               if (b.FeedForward.weights.size() == 2) {
                 L["ffn_w1"] = fw[0];
                 L["ffn_b1"] = fb[0];
                 L["ffn_w2"] = fw[1];
                 L["ffn_b2"] = fb[1];
               }
               L["ffn_weights"] = fw;
               L["ffn_biases"] = fb;
               L["ffn_activations"] = fa;
               layers.append(L);
             }
             w["layers"] = layers;
             return w;
           })
      .def("Forward", [](LanguageModel &lm, py::object ids) { return to_numpy(lm.Forward(ids_from(ids))); })
      .def("ForwardContinuous",
           [](LanguageModel &lm, py::object x) {
             auto X = mat(x);
             return to_numpy(lm.Forward(X.view));
           })
      .def("PredictNext",
           [](LanguageModel &lm, py::object x) {
             auto X = mat(x);
             return lm.PredictNext(X.view);
           })
      .def("Generate",
           [](LanguageModel &lm, py::object prompt, int maxNew, float temperature, bool greedy, uint64_t seed) {
             return lm.Generate(ids_from(prompt), maxNew, temperature, greedy, seed);
           },
           py::arg("prompt"), py::arg("maxNewTokens"), py::arg("temperature") = 1.0f,
           py::arg("greedy") = true, py::arg("seed") = 0);

  py::class_<TrainingConfig>(m, "TrainingConfig")
      .def(py::init<>())
      .def_readwrite("LearningRate", &TrainingConfig::LearningRate)
      .def_readwrite("BatchSize", &TrainingConfig::BatchSize)
      .def_readwrite("Epochs", &TrainingConfig::Epochs)
      .def_readwrite("UseGradientClipping", &TrainingConfig::UseGradientClipping)
      .def_readwrite("GradientClipThreshold", &TrainingConfig::GradientClipThreshold)
      .def_readwrite("UseLearningRateDecay", &TrainingConfig::UseLearningRateDecay)
      .def_readwrite("LearningRateDecay", &TrainingConfig::LearningRateDecay)
      .def_readwrite("ValidationInterval", &TrainingConfig::ValidationInterval)
      .def_readwrite("Verbose", &TrainingConfig::Verbose);

  auto seqs_from = [](const py::object &o) {
    std::vector<std::vector<int>> out;
    for (py::handle h : o) {
      I32 a = I32::ensure(py::reinterpret_borrow<py::object>(h));
      if (!a || a.ndim() != 1) throw ArgumentException("each sequence must be a 1-D int array", "batch");
      out.emplace_back(a.data(), a.data() + a.size());
    }
    return out;
  };
  // Windows [len, F], regression targets [len, O] and class-id arrays; None
  // entries become empty (the trainer skips those windows).
  auto cont_from = [](const py::object &inputs, const py::object &reg, const py::object &cls,
                      std::vector<Matrix> &xs, std::vector<Matrix> &rs, std::vector<std::vector<int>> &cs) {
    auto mats = [](const py::object &o, std::vector<Matrix> &out) {
      for (py::handle h : o) {
        py::object ob = py::reinterpret_borrow<py::object>(h);
        out.push_back(ob.is_none() ? Matrix() : from_numpy(ob));
      }
    };
    mats(inputs, xs);
    if (!reg.is_none()) mats(reg, rs);
    if (!cls.is_none())
      for (py::handle h : cls) {
        py::object ob = py::reinterpret_borrow<py::object>(h);
        cs.push_back(ob.is_none() ? std::vector<int>() : ids_from(ob));
      }
  };
  auto flat_dict = [](DeviceTrainer &t, const std::vector<float> &flat) {
    py::dict d;
    for (size_t i = 0; i < t.names().size(); ++i) {
      const auto &o = t.offsets()[i];
      py::array_t<float> a((py::ssize_t)o.second);
      std::memcpy(a.mutable_data(), flat.data() + o.first, o.second * sizeof(float));
      d[py::str(t.names()[i])] = a;
    }
    return d;
  };
  py::class_<TransformerTrainer>(m, "TransformerTrainer")
      .def(py::init<LanguageModel &, const TrainingConfig &>(), py::arg("model"), py::arg("config"),
           py::keep_alive<1, 2>())
      .def("TrainBatch",
           [seqs_from](TransformerTrainer &t, py::object batch, float lr) {
             auto b = seqs_from(batch);
             return nogil([&] { return t.TrainBatch(b, lr); });
           },
           py::arg("batch"), py::arg("learningRate"))
      .def("Train",
           [seqs_from](TransformerTrainer &t, py::object seqs, uint64_t seed, py::object val) {
             auto b = seqs_from(seqs);
             std::vector<std::vector<int>> v;
             if (!val.is_none()) v = seqs_from(val);
             return nogil([&] { return t.Train(b, seed, val.is_none() ? nullptr : &v); });
           },
           py::arg("sequences"), py::arg("seed") = 0, py::arg("validationSequences") = py::none())
      .def("TrainBatchContinuous",
           [cont_from](TransformerTrainer &t, py::object inputs, py::object reg, py::object cls, float lr) {
             std::vector<Matrix> xs, rs;
             std::vector<std::vector<int>> cs;
             cont_from(inputs, reg, cls, xs, rs, cs);
             return nogil([&] {
               return t.TrainBatchContinuous(xs, reg.is_none() ? nullptr : &rs, cls.is_none() ? nullptr : &cs, lr);
             });
           },
           py::arg("inputs"), py::arg("regressionTargets") = py::none(), py::arg("classTargets") = py::none(),
           py::arg("learningRate") = 0.0001f)
      .def("TrainContinuous",
           [cont_from](TransformerTrainer &t, py::object inputs, py::object reg, py::object cls, uint64_t seed) {
             std::vector<Matrix> xs, rs;
             std::vector<std::vector<int>> cs;
             cont_from(inputs, reg, cls, xs, rs, cs);
             return nogil([&] {
               return t.TrainContinuous(xs, reg.is_none() ? nullptr : &rs, cls.is_none() ? nullptr : &cs, seed);
             });
           },
           py::arg("inputs"), py::arg("regressionTargets") = py::none(), py::arg("classTargets") = py::none(),
           py::arg("seed") = 0)
      .def("Validate",
           [seqs_from](TransformerTrainer &t, py::object seqs) {
             auto b = seqs_from(seqs);
             return nogil([&] { return t.Validate(b); });
           },
           py::arg("validationSequences"))
      .def("ValidateContinuous",
           [cont_from](TransformerTrainer &t, py::object inputs, py::object reg, py::object cls) {
             std::vector<Matrix> xs, rs;
             std::vector<std::vector<int>> cs;
             cont_from(inputs, reg, cls, xs, rs, cs);
             return nogil([&] {
               return t.ValidateContinuous(xs, reg.is_none() ? nullptr : &rs, cls.is_none() ? nullptr : &cs);
             });
           },
           py::arg("inputs"), py::arg("regressionTargets") = py::none(), py::arg("classTargets") = py::none())
      .def_property_readonly("last_norm", &TransformerTrainer::last_norm)
      .def_property_readonly("validation_losses", &TransformerTrainer::validation_losses)
      .def("gradients",
           // the gradients the last update applied (after the 1/validCount and
           // clipping scales), flat names as DeviceTrainer.gradients()
           [](const TransformerTrainer &t) {
             const auto &g = t.gradients();
             py::dict d;
             if (!g.InputProjectionBiasGrad.empty()) {
               d["input_proj"] = to_numpy(g.InputProjectionGrad);
               d["input_bias"] = vec_to_numpy(g.InputProjectionBiasGrad);
             } else {
               d["token_embedding"] = to_numpy(g.TokenEmbeddingGrad);
             }
             d["out_proj"] = to_numpy(g.OutputProjectionGrad);
             d["out_bias"] = vec_to_numpy(g.OutputBiasGrad);
             for (size_t i = 0; i < g.AttentionGrads.size(); ++i) {
               const auto &a = g.AttentionGrads[i];
               const std::string p = "layers." + std::to_string(i) + ".";
               d[py::str(p + "wq")] = to_numpy(a.WQ_Grad);
               d[py::str(p + "wk")] = to_numpy(a.WK_Grad);
               d[py::str(p + "wv")] = to_numpy(a.WV_Grad);
               d[py::str(p + "wo")] = to_numpy(a.WO_Grad);
               d[py::str(p + "bq")] = vec_to_numpy(a.BiasQ_Grad);
               d[py::str(p + "bk")] = vec_to_numpy(a.BiasK_Grad);
               d[py::str(p + "bv")] = vec_to_numpy(a.BiasV_Grad);
               d[py::str(p + "bo")] = vec_to_numpy(a.BiasO_Grad);
               d[py::str(p + "ln1_g")] = vec_to_numpy(g.LN1Grads[i].GammaGrad);
               d[py::str(p + "ln1_b")] = vec_to_numpy(g.LN1Grads[i].BetaGrad);
               d[py::str(p + "ln2_g")] = vec_to_numpy(g.LN2Grads[i].GammaGrad);
               d[py::str(p + "ln2_b")] = vec_to_numpy(g.LN2Grads[i].BetaGrad);
               const auto &fw = t.ffn_weight_gradients()[i];
               const auto &fb = t.ffn_bias_gradients()[i];
               for (size_t l = 0; l < fw.size(); ++l) {
                 d[py::str(p + "ffn_w" + std::to_string(l + 1))] = to_numpy(fw[l]);
                 d[py::str(p + "ffn_b" + std::to_string(l + 1))] = vec_to_numpy(fb[l]);
               }
             }
             return d;
           });

  py::class_<DeviceTrainer>(m, "DeviceTrainer")
      .def(py::init<const LanguageModel &, const TrainingConfig &, int, int, int>(), py::arg("model"),
           py::arg("config"), py::arg("batch_capacity"), py::arg("seq_capacity"), py::arg("device") = 0)
      .def("TrainBatch",
           [seqs_from](DeviceTrainer &t, py::object batch, float lr) {
             auto b = seqs_from(batch);
             py::gil_scoped_release nogil;
             return t.TrainBatch(b, lr);
           },
           py::arg("batch"), py::arg("learningRate"))
      .def("Train",
           [seqs_from](DeviceTrainer &t, py::object seqs, uint64_t seed) {
             auto b = seqs_from(seqs);
             py::gil_scoped_release nogil;
             return t.Train(b, seed);
           },
           py::arg("sequences"), py::arg("seed") = 0)
      .def("TrainBatchContinuous",
           [cont_from](DeviceTrainer &t, py::object inputs, py::object reg, py::object cls, float lr) {
             std::vector<Matrix> xs, rs;
             std::vector<std::vector<int>> cs;
             cont_from(inputs, reg, cls, xs, rs, cs);
             py::gil_scoped_release nogil;
             return t.TrainBatchContinuous(xs, rs, cs, lr);
           },
           py::arg("inputs"), py::arg("regressionTargets") = py::none(), py::arg("classTargets") = py::none(),
           py::arg("learningRate") = 1e-4f)
      .def("TrainContinuous",
           [cont_from](DeviceTrainer &t, py::object inputs, py::object reg, py::object cls, uint64_t seed) {
             std::vector<Matrix> xs, rs;
             std::vector<std::vector<int>> cs;
             cont_from(inputs, reg, cls, xs, rs, cs);
             py::gil_scoped_release nogil;
             return t.TrainContinuous(xs, rs, cs, seed);
           },
           py::arg("inputs"), py::arg("regressionTargets") = py::none(), py::arg("classTargets") = py::none(),
           py::arg("seed") = 0)
      .def("CopyWeightsTo", &DeviceTrainer::CopyWeightsTo, py::arg("model"))
      .def("weights", [flat_dict](DeviceTrainer &t) { return flat_dict(t, t.weights_flat()); })
      .def("gradients", [flat_dict](DeviceTrainer &t) { return flat_dict(t, t.gradients_flat()); })
      .def_property_readonly("last_norm", &DeviceTrainer::last_norm)
      .def("time_step",
           // Whole training steps on one fixed bucket (tokens [batch, seqLen + 1])
           // resident in HBM: mean ms of `steps` steps after `warmup`, host clock
           // with the stream synchronised on both sides.
           [](DeviceTrainer &t, py::object tokens, float lr, int steps, int warmup) {
             I32 a = I32::ensure(tokens);
             if (!a || a.ndim() != 2) throw ArgumentException("tokens must be [batch, seqLen + 1]", "tokens");
             py::gil_scoped_release nogil;
             t.load_batch(a.data(), (int)a.shape(0), (int)a.shape(1));
             for (int i = 0; i < warmup; ++i) t.step_loaded(lr);
             t.synchronize();
             const auto t0 = std::chrono::steady_clock::now();
             for (int i = 0; i < steps; ++i) t.step_loaded(lr);
             t.synchronize();
             const auto t1 = std::chrono::steady_clock::now();
             return std::chrono::duration<double, std::milli>(t1 - t0).count() / std::max(steps, 1);
           },
           py::arg("tokens"), py::arg("learningRate"), py::arg("steps") = 5, py::arg("warmup") = 2)
      .def("time_step_continuous",
           // time_step for a regression model: inputs [batch, seqLen + 1, F],
           // targets [batch, seqLen + 1, OutputDim]
           [](DeviceTrainer &t, py::object inputs, py::object targets, float lr, int steps, int warmup) {
             F32 x = F32::ensure(inputs), y = F32::ensure(targets);
             if (!x || !y || x.ndim() != 3 || y.ndim() != 3 || x.shape(0) != y.shape(0) || x.shape(1) != y.shape(1))
               throw ArgumentException("inputs [batch, T, F] and targets [batch, T, O] expected", "inputs");
             py::gil_scoped_release nogil;
             t.load_batch_continuous(x.data(), y.data(), (int)x.shape(0), (int)x.shape(1));
             for (int i = 0; i < warmup; ++i) t.step_loaded(lr);
             t.synchronize();
             const auto t0 = std::chrono::steady_clock::now();
             for (int i = 0; i < steps; ++i) t.step_loaded(lr);
             t.synchronize();
             const auto t1 = std::chrono::steady_clock::now();
             return std::chrono::duration<double, std::milli>(t1 - t0).count() / std::max(steps, 1);
           },
           py::arg("inputs"), py::arg("targets"), py::arg("learningRate"), py::arg("steps") = 5,
           py::arg("warmup") = 2);

  py::class_<DeviceLanguageModel>(m, "DeviceLanguageModel")
      .def(py::init<const LanguageModel &, int, int>(), py::arg("model"), py::arg("batch_capacity"),
           py::arg("device") = 0)
      .def("Forward",
           [](DeviceLanguageModel &d, py::object ids) {
             I32 a = I32::ensure(ids);
             if (!a || a.ndim() != 2) throw ArgumentException("ids must be [batch, seqLen]", "ids");
             std::vector<int> v(a.data(), a.data() + a.size());
             return to_numpy(d.Forward(v, (int)a.shape(0), (int)a.shape(1)));
           })
      .def("ForwardContinuous",
           [](DeviceLanguageModel &d, py::object x, int batch, int seqLen) {
             auto X = mat(x);
             return to_numpy(d.ForwardContinuous(X.view, batch, seqLen));
           })
      .def("Layers",
           // The decoder blocks alone on embeddings x [batch * seqLen, D]
           // (the c3 stack's input): uploads x, runs every block in place on
           // the device and returns the result.
           [](DeviceLanguageModel &d, py::object x, int batch, int seqLen) {
             auto X = mat(x);
             if (X.view.null() || (long long)X.view.rows != (long long)batch * seqLen)
               throw ArgumentException("x must be [batch * seqLen, D]", "x");
             if (batch <= 0 || batch > d.batch_capacity()) throw ArgumentOutOfRangeException("batch");
             auto chk = [](int rc) {
               if (rc != CDML_OK) throw InvalidOperationException(cdml_last_error());
             };
             Matrix out(X.view.rows, X.view.cols);
             void *dx = nullptr;
             const size_t bytes = (size_t)X.view.rows * X.view.cols * sizeof(float);
             chk(cdml_malloc(&dx, bytes));
             try {
               py::gil_scoped_release nogil;
               chk(cdml_memcpy_h2d_async(dx, X.view.data, bytes, d.stream()));
               d.layers_device(static_cast<float *>(dx), batch, seqLen);
               chk(cdml_memcpy_d2h_async(out.ptr(), dx, bytes, d.stream()));
               d.synchronize();
             } catch (...) {
               cdml_free(dx);
               throw;
             }
             cdml_free(dx);
             return to_numpy(std::move(out));
           },
           py::arg("x"), py::arg("batch"), py::arg("seqLen"))
      .def_readwrite("use_graphs", &DeviceLanguageModel::use_graphs)
      .def_readwrite("use_fused_decode", &DeviceLanguageModel::use_fused_decode)
      .def_property_readonly("fused_decode_available", &DeviceLanguageModel::fused_decode_available)
      .def("GenerateGreedy",
           [](DeviceLanguageModel &d, py::object prompts, int maxNew) {
             I32 a = I32::ensure(prompts);
             if (!a || a.ndim() != 2) throw ArgumentException("prompts must be [batch, promptLen]", "prompts");
             std::vector<int> v(a.data(), a.data() + a.size());
             int total = 0;
             std::vector<int> out = d.GenerateGreedy(v, (int)a.shape(0), (int)a.shape(1), maxNew, &total);
             py::array_t<int> r({(py::ssize_t)a.shape(0), (py::ssize_t)total});
             std::memcpy(r.mutable_data(), out.data(), out.size() * sizeof(int));
             return r;
           })
      .def("time_forward",
           // Device-resident forward of `batch` sequences of `seqLen` inputs
           // that are already in HBM: returns the mean ms of `steps` launches
           // (HIP events on the model's stream) after `warmup` untimed ones.
           [](DeviceLanguageModel &d, py::object inputs, int batch, int seqLen, int steps, int warmup,
              bool continuous) {
             void *din = nullptr, *dout = nullptr;
             auto chk = [](int rc) {
               if (rc != CDML_OK) throw InvalidOperationException(cdml_last_error());
             };
             if (batch <= 0 || batch > d.batch_capacity()) throw ArgumentOutOfRangeException("batch");
             py::array arr = inputs;
             const size_t need = (size_t)batch * seqLen * (continuous ? sizeof(float) : sizeof(int));
             if (!(arr.flags() & py::array::c_style) || (size_t)arr.nbytes() < need ||
                 arr.itemsize() != 4)
               throw ArgumentException("inputs must be a C-contiguous 4-byte array of batch * seqLen rows",
                                       "inputs");
             chk(cdml_malloc(&din, arr.nbytes()));
             chk(cdml_memcpy_h2d_async(din, arr.data(), arr.nbytes(), d.stream()));
             chk(cdml_malloc(&dout, (size_t)batch * seqLen * d.output_dim() * sizeof(float)));
             cdml_event e0, e1;
             chk(cdml_event_create(&e0));
             chk(cdml_event_create(&e1));
             float ms = 0.f;
             {
               py::gil_scoped_release nogil;
               for (int i = 0; i < warmup; ++i)
                 d.forward_device(continuous ? nullptr : static_cast<int *>(din),
                                  continuous ? static_cast<float *>(din) : nullptr, batch, seqLen,
                                  static_cast<float *>(dout));
               d.synchronize();
               chk(cdml_event_record(e0, d.stream()));
               for (int i = 0; i < steps; ++i)
                 d.forward_device(continuous ? nullptr : static_cast<int *>(din),
                                  continuous ? static_cast<float *>(din) : nullptr, batch, seqLen,
                                  static_cast<float *>(dout));
               chk(cdml_event_record(e1, d.stream()));
               chk(cdml_event_elapsed_ms(e0, e1, &ms));
             }
             cdml_event_destroy(e0);
             cdml_event_destroy(e1);
             cdml_free(din);
             cdml_free(dout);
             return ms / std::max(steps, 1);
           },
           py::arg("inputs"), py::arg("batch"), py::arg("seqLen"), py::arg("steps") = 10,
           py::arg("warmup") = 2, py::arg("continuous") = false)
      .def("time_layers",
           // The decoder blocks alone on embeddings x [batch * seqLen, D]
           // resident in HBM: mean ms of `steps` passes after `warmup`.
           [](DeviceLanguageModel &d, py::object x, int batch, int seqLen, int steps, int warmup) {
             auto X = mat(x);
             if (X.view.null() || X.view.rows != batch * seqLen)
               throw ArgumentException("x must be [batch * seqLen, D]", "x");
             if (batch <= 0 || batch > d.batch_capacity()) throw ArgumentOutOfRangeException("batch");
             auto chk = [](int rc) {
               if (rc != CDML_OK) throw InvalidOperationException(cdml_last_error());
             };
             void *dx = nullptr;
             const size_t bytes = (size_t)X.view.rows * X.view.cols * sizeof(float);
             chk(cdml_malloc(&dx, bytes));
             chk(cdml_memcpy_h2d_async(dx, X.view.data, bytes, d.stream()));
             cdml_event e0, e1;
             chk(cdml_event_create(&e0));
             chk(cdml_event_create(&e1));
             float ms = 0.f;
             {
               py::gil_scoped_release nogil;
               for (int i = 0; i < warmup; ++i) d.layers_device(static_cast<float *>(dx), batch, seqLen);
               d.synchronize();
               chk(cdml_event_record(e0, d.stream()));
               for (int i = 0; i < steps; ++i) d.layers_device(static_cast<float *>(dx), batch, seqLen);
               chk(cdml_event_record(e1, d.stream()));
               chk(cdml_event_elapsed_ms(e0, e1, &ms));
             }
             cdml_event_destroy(e0);
             cdml_event_destroy(e1);
             cdml_free(dx);
             return ms / std::max(steps, 1);
           },
           py::arg("x"), py::arg("batch"), py::arg("seqLen"), py::arg("steps") = 3, py::arg("warmup") = 1);
}

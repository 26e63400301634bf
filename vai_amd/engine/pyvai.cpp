// pyvai.cpp -- Python bindings of the engine, shaped like the reference's
// pyvai (/root/reference/python/bindings: NeuralNet, Tensor, nodes.LinearNode
// with in_dim / out_dim / accept_residual / residual_order / epilogue /
// scalar_scale / split_size, ConvolutionNode, GatedMulNode), so node tests
// read like /root/reference/python/tests/node_check.py.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "graph-flow.h"
#include "neural-net.h"
#include "nodes.h"

namespace py = pybind11;
using namespace vai;

namespace {

Tensor fromNumpy(py::array arr, py::object dtype)
{
    py::array a = py::array::ensure(arr, py::array::c_style);
    std::vector<uint32_t> shape(a.shape(), a.shape() + a.ndim());
    if (shape.empty()) shape = {1};
    const bool isHalf = a.dtype().is(py::dtype("float16"));
    Dtype want = isHalf ? Dtype::Fp16 : Dtype::Fp32;
    if (!dtype.is_none()) want = dtype.cast<Dtype>();
    Tensor t(shape, want);
    if (isHalf) {
        if (want == Dtype::Fp16) t.setData(static_cast<const uint16_t*>(a.data()));
        else {
            std::vector<float> f(a.size());
            convertDtype(a.data(), Dtype::Fp16, f.data(), Dtype::Fp32, a.size());
            t.setFloats(f.data());
        }
    } else {
        py::array_t<float, py::array::c_style | py::array::forcecast> f(a);
        t.setFloats(f.data());
    }
    return t;
}

py::array toNumpy(Tensor& t)
{
    std::vector<ssize_t> shape(t.shape().begin(), t.shape().end());
    if (t.dtype() == Dtype::Fp16) {
        const uint16_t* p = t.getData<uint16_t>();
        py::array out(py::dtype("float16"), shape);
        std::memcpy(out.mutable_data(), p, t.numBytes());
        return out;
    }
    const float* p = t.getData<float>();
    py::array_t<float> out(shape);
    std::memcpy(out.mutable_data(), p, t.numBytes());
    return out;
}

// A Python-side flow: (node, inSlot, outSlot), for `a - b`, `"s"/n`, `n/"s"`.
struct PyFlow {
    Node* node;
    std::string in, out;
};

PyFlow flowOf(py::object o)
{
    if (py::isinstance<PyFlow>(o)) return o.cast<PyFlow>();
    return PyFlow{o.cast<Node*>(), "in0", "out0"};
}

PyFlow connect(py::object a, py::object b)
{
    PyFlow fa = flowOf(a), fb = flowOf(b);
    NodeSlot::connect(fa.node->slot(fa.out), fb.node->slot(fb.in));
    return fb;
}

// NeuralNet subclassable from Python; construction makes it current so nodes
// built in __init__ bind to it, as in the reference.
class PyNet : public NeuralNet
{
public:
    using NeuralNet::NeuralNet;
    DtypeKey key() { return dtypeKey(); }
};

}   // namespace

static vai::node::CausalBlockEnd block_ends(const std::vector<uint32_t>& ends)
{
    vai::node::CausalBlockEnd e{};
    if (ends.size() > e.size()) throw std::invalid_argument("at most 31 block ends");
    std::copy(ends.begin(), ends.end(), e.begin());
    return e;
}

PYBIND11_MODULE(_pyvai, m)
{
    m.doc() = "vai_amd engine: NeuralNet / Tensor / nodes on MI355X kernels";

    py::enum_<Dtype>(m, "Dtype").value("F32", Dtype::Fp32).value("F16", Dtype::Fp16);
    py::enum_<Epilogue>(m, "Epilogue")
        .value("NONE", Epilogue::None).value("RELU", Epilogue::Relu).value("GELU", Epilogue::Gelu)
        .value("GELU_TANH", Epilogue::GeluTanh).value("SILU", Epilogue::Silu).value("SIGMOID", Epilogue::Sigmoid);
    py::enum_<ResidualOrder>(m, "ResidualOrder")
        .value("AFTER_EPILOGUE", ResidualOrder::AfterEpilogue)
        .value("BEFORE_EPILOGUE", ResidualOrder::BeforeEpilogue);

    py::class_<Tensor>(m, "Tensor")
        .def_static("from_numpy", &fromNumpy, py::arg("array"), py::arg("dtype") = py::none())
        .def("to_numpy", &toNumpy)
        .def_property_readonly("shape", [](const Tensor& t) { return t.shape(); })
        .def_property_readonly("dtype", &Tensor::dtype)
        .def("num_elements", &Tensor::numElements)
        .def("valid", &Tensor::validShape);

    py::class_<PyFlow>(m, "Flow")
        .def("__sub__", [](PyFlow& a, py::object b) { return connect(py::cast(a), b); })
        .def("__truediv__", [](PyFlow f, const std::string& s) { f.out = s; return f; });

    py::class_<Node>(m, "Node")
        .def("__getitem__", [](Node& n, const std::string& s) { return n[s]; })
        .def("__setitem__", [](Node& n, const std::string& s, const Tensor& t) { n[s] = t; })
        .def("__sub__", [](py::object a, py::object b) { return connect(a, b); })
        .def("__rtruediv__", [](Node& n, const std::string& s) { return PyFlow{&n, s, "out0"}; })
        .def("__truediv__", [](Node& n, const std::string& s) { return PyFlow{&n, "in0", s}; })
        .def_property_readonly("kind", [](Node& n) { return std::string(n.kind()); });

    py::class_<InputNode, Node>(m, "InputNode");
    py::class_<OutputNode, Node>(m, "OutputNode");

    py::class_<PyNet>(m, "NeuralNet")
        .def(py::init([](Dtype w, Dtype o, bool graph, bool fuse, int device) {
                 NeuralNetConfig c;
                 c.wDefaultDtype = w;
                 c.oDefaultDtype = o;
                 c.useGraph = graph;
                 c.fuseGatedLinear = fuse;
                 c.device = device;
                 return std::make_unique<PyNet>(c);
             }),
             py::arg("w_default_dtype") = Dtype::Fp16, py::arg("o_default_dtype") = Dtype::Fp32,
             py::arg("use_graph") = true, py::arg("fuse_gated_linear") = true, py::arg("device") = 0)
        .def("input", &PyNet::input, py::return_value_policy::reference_internal)
        .def("output", &PyNet::output, py::return_value_policy::reference_internal)
        .def("sync", &PyNet::sync)
        .def_property_readonly("record_count", &PyNet::recordCount)
        .def_property_readonly("submit_count", &PyNet::submitCount)
        .def("set_o_dtype", [](PyNet& net, Node& n, Dtype d) { n.setODtype(d, net.key()); })
        .def("set_acc_dtype", [](PyNet& net, node::Linear& l, Dtype d) { l.setAccDtype(d, net.key()); })
        .def("__call__", [](PyNet& net, py::kwargs kw) {
            TensorDict in;
            for (auto item : kw) in[item.first.cast<std::string>()] = item.second.cast<Tensor>();
            std::map<std::string, Tensor> outs;
            TensorRefDict refs;
            for (const auto& name : net.outputNames()) outs[name] = Tensor();
            for (auto& [s, t] : outs) refs[s] = &t;
            net(in, refs);
            if (outs.size() == 1) return py::cast(outs.begin()->second);
            py::dict d;
            for (auto& [s, t] : outs) d[py::str(s)] = t;
            return py::object(d);
        });

    auto nodes = m.def_submodule("nodes");
    py::class_<node::Linear, Node>(nodes, "LinearNode")
        .def(py::init([](uint32_t in_dim, uint32_t out_dim, bool accept_residual, ResidualOrder residual_order,
                         Epilogue epilogue, float scalar_scale, uint32_t split_size) {
                 node::Linear::Config c{in_dim, out_dim};
                 c.acceptResidual = accept_residual;
                 c.residualOrder = residual_order;
                 c.epilogue = epilogue;
                 c.scalarScale = scalar_scale;
                 c.splitSize = split_size;
                 return std::make_unique<node::Linear>(c);
             }),
             py::arg("in_dim"), py::arg("out_dim"), py::arg("accept_residual") = false,
             py::arg("residual_order") = ResidualOrder::AfterEpilogue, py::arg("epilogue") = Epilogue::None,
             py::arg("scalar_scale") = 1.0f, py::arg("split_size") = 0)
        .def_property_readonly("plan", &node::Linear::plan)
        .def_property_readonly("split_count", &node::Linear::splitCount)
        .def_property_readonly("fused", [](node::Linear& l) { return l.fusedGate() != nullptr; })
        .def("has_bias", &node::Linear::hasBias);
    py::class_<node::GatedMul, Node>(nodes, "GatedMulNode")
        .def(py::init([](Epilogue activation) {
                 return std::make_unique<node::GatedMul>(node::GatedMul::Config{activation});
             }),
             py::arg("activation") = Epilogue::Silu);
    py::class_<node::Convolution, Node>(nodes, "ConvolutionNode")
        .def(py::init([](uint32_t in_channels, uint32_t out_channels, uint32_t kernel_size, uint32_t stride,
                         bool accept_residual, ResidualOrder residual_order, Epilogue epilogue) {
                 node::Convolution::Config c{in_channels, out_channels, kernel_size, stride};
                 c.acceptResidual = accept_residual;
                 c.residualOrder = residual_order;
                 c.epilogue = epilogue;
                 return std::make_unique<node::Convolution>(c);
             }),
             py::arg("in_channels"), py::arg("out_channels"), py::arg("kernel_size"), py::arg("stride") = 1,
             py::arg("accept_residual") = false, py::arg("residual_order") = ResidualOrder::AfterEpilogue,
             py::arg("epilogue") = Epilogue::None);
    py::class_<node::AttentionScores, Node>(nodes, "AttentionScoresNode")
        .def(py::init([](uint32_t num_q_heads, uint32_t head_dim, uint32_t num_kv_heads, bool causal, uint32_t span,
                         float scale) {
                 node::AttentionScores::Config c{num_q_heads, num_kv_heads, head_dim, causal, span, scale};
                 return std::make_unique<node::AttentionScores>(c);
             }),
             py::arg("num_q_heads"), py::arg("head_dim"), py::arg("num_kv_heads") = 0, py::arg("causal") = true,
             py::arg("span") = 0, py::arg("scale") = 0.0f)
        .def("set_causal_mask", [](node::AttentionScores& n, uint32_t bits, std::vector<uint32_t> ends, uint32_t span) {
                 n.setCausalMask(node::CausalMask::make(bits, block_ends(ends), span));
             }, py::arg("bits"), py::arg("block_end") = std::vector<uint32_t>{}, py::arg("span") = 0);
    py::class_<node::Attention, Node>(nodes, "AttentionNode")
        .def(py::init([](uint32_t num_q_heads, uint32_t head_dim, uint32_t num_kv_heads, uint32_t kv_cache_size,
                         py::object kv_cache_dtype, bool kv_cache_ring) {
                 node::Attention::Config c{.headDim = head_dim, .numQHeads = num_q_heads, .numKVHeads = num_kv_heads,
                                           .kvCacheSize = kv_cache_size,
                                           .kvCacheDtype = kv_cache_dtype.is_none() ? Dtype::None
                                                                                    : kv_cache_dtype.cast<Dtype>(),
                                           .kvCacheRing = kv_cache_ring};
                 return std::make_unique<node::Attention>(c);
             }),
             py::arg("num_q_heads"), py::arg("head_dim"), py::arg("num_kv_heads") = 0, py::arg("kv_cache_size") = 0,
             py::arg("kv_cache_dtype") = py::none(), py::arg("kv_cache_ring") = false)
        .def("set_kv_cache_counter", [](node::Attention& n, uintptr_t ptr) {
                 n.setKvCacheCounter(reinterpret_cast<const uint32_t*>(ptr));
             }, py::arg("device_ptr"))
        .def_property_readonly("kv_cache_size", [](node::Attention& n) { return n.config_.kvCacheSize; })
        .def("set_causal_mask", [](node::Attention& n, uint32_t bits, std::vector<uint32_t> ends, uint32_t span) {
                 n.setCausalMask(node::CausalMask::make(bits, block_ends(ends), span));
             }, py::arg("bits"), py::arg("block_end") = std::vector<uint32_t>{}, py::arg("span") = 0);
}

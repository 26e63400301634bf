// neural-net.cpp -- ordering, parameter upload, buffer binding, HIP-graph
// record/replay and the Linear -> GatedMul fusion.
#include "neural-net.h"

#include <algorithm>
#include <deque>
#include <set>
#include <stdexcept>

#include "../../include/vai_amd.h"
#include "graph-flow.h"
#include "nodes.h"

namespace vai {

static void check(vai_status st, const char* what)
{
    if (st != VAI_OK) throw std::runtime_error(std::string(what) + ": " + vai_status_string(st));
}

void NodeSlot::connect(NodeSlot& a, NodeSlot& b)
{
    require(a.type_ == output && b.type_ == input, "connect: an output slot feeds an input slot");
    for (NodeSlot* s : a.connections_)
        if (s == &b) return;
    a.connections_.push_back(&b);
    b.connections_.push_back(&a);
}

void NodeSlot::disconnect(NodeSlot& a, NodeSlot& b)
{
    std::erase(a.connections_, &b);
    std::erase(b.connections_, &a);
}

Node::Node() : ownedNet_(NeuralNet::current())
{
    require(ownedNet_ != nullptr, "a Node must be constructed while its NeuralNet is being built");
}

Dtype Node::wDefaultDtype() const { return ownedNet_->config().wDefaultDtype; }
Dtype Node::oDefaultDtype() const { return ownedNet_->config().oDefaultDtype; }
BufferPool& Node::bufferPool() const { return ownedNet_->bufferPool(); }
Dtype Node::outputDtype() const { return oDtype_ == Dtype::None ? oDefaultDtype() : oDtype_; }

NodeSlot& Node::slot(const std::string& name)
{
    auto it = slots_.find(name);
    require(it != slots_.end(), std::string("no slot named ") + name);
    return it->second;
}

InputNode::InputNode()
{
    addSlot("in0", NodeSlot::none);
    addSlot("out0", NodeSlot::output);
}

OutputNode::OutputNode() { addSlot("in0", NodeSlot::input); }

void OutputNode::prepare() {}

NeuralNet::NeuralNet(const NeuralNetConfig& config) : config_(config)
{
    require(config_.wDefaultDtype != Dtype::None && config_.oDefaultDtype != Dtype::None,
            "NeuralNetConfig: default dtypes must not be None");
    currentNet_ = this;
    bufferPool_ = config_.bufferPool ? config_.bufferPool
                                     : std::make_shared<BufferPool>(config_.bufferPoolLogLevel);
}

void* NeuralNet::stream()
{
    // Created on first use, so wiring and shape errors surface without a GPU.
    if (!stream_) {
        check(vai_set_device(config_.device), "set_device");
        vai_stream_t s = nullptr;
        check(vai_stream_create(&s), "stream_create");
        stream_ = s;
    }
    return stream_;
}

NeuralNet::~NeuralNet()
{
    if (stream_) vai_stream_sync((vai_stream_t)stream_);
    destroyGraph();
    if (stream_) vai_stream_destroy((vai_stream_t)stream_);
    if (currentNet_ == this) currentNet_ = nullptr;
}

void NeuralNet::destroyGraph()
{
    if (graph_) vai_graph_destroy((vai_graph_t)graph_);
    graph_ = nullptr;
}

void NeuralNet::sync()
{
    if (submitCount_) check(vai_stream_sync((vai_stream_t)stream_), "sync");
}

void NeuralNet::sortNodes()
{
    // Every node reachable from the inputs through the wiring, plus nodes on
    // the way to the outputs.
    std::set<Node*> seen;
    std::deque<Node*> work;
    for (auto& [name, in] : inputs_) { work.push_back(&in); seen.insert(&in); }
    for (auto& [name, out] : outputs_) { work.push_back(&out); seen.insert(&out); }
    while (!work.empty()) {
        Node* n = work.front();
        work.pop_front();
        for (auto& [sname, s] : n->slots_)
            for (NodeSlot* c : s.connections_) {
                Node* m = &c->parentNode();
                if (seen.insert(m).second) work.push_back(m);
            }
    }
    // Kahn: a node is ready once every producer of its input slots is placed.
    std::map<Node*, int> indeg;
    for (Node* n : seen) {
        int d = 0;
        for (auto& [sname, s] : n->slots_)
            if (s.type_ == NodeSlot::input) {
                if (s.connections_.size() > 1)
                    throw std::runtime_error("input slot " + sname + " has more than one producer");
                d += int(s.connections_.size());
            }
        indeg[n] = d;
    }
    std::deque<Node*> ready;
    for (auto& [n, d] : indeg)
        if (d == 0) ready.push_back(n);
    sortedNodes_.clear();
    while (!ready.empty()) {
        Node* n = ready.front();
        ready.pop_front();
        sortedNodes_.push_back(n);
        for (auto& [sname, s] : n->slots_)
            if (s.type_ == NodeSlot::output)
                for (NodeSlot* c : s.connections_)
                    if (--indeg[&c->parentNode()] == 0) ready.push_back(&c->parentNode());
    }
    if (sortedNodes_.size() != seen.size()) throw std::runtime_error("the graph has a cycle");
}

void NeuralNet::uploadModelParams()
{
    for (Node* n : sortedNodes_)
        for (auto& [name, s] : n->slots_) {
            if (s.type_ != NodeSlot::persistent) continue;
            Tensor& t = s.value_;
            if (!t.validShape() || !t.hasHostData()) continue;
            if (t.data_->hostUploaded_ && t.gpuBufferBound()) continue;
            if (!t.gpuBufferBound()) t.bindBuffer(bufferPool_->requestBuffer(t.numBytes()));
            t.upload(stream());
        }
}

void NeuralNet::prepareInputs()
{
    for (InputNode* in : activeInputs_) {
        Tensor& t = (*in)["in0"];
        require(t.validShape(), "input tensor has no shape");
        if (t.gpuBufferBound() && !t.hasHostData()) continue;   // already device data
        if (!t.gpuBufferBound()) {
            // keep the previous forward's buffer while the shape holds, so a
            // recorded graph stays valid
            Tensor& prev = (*in)["out0"];
            if (prev.gpuBufferBound() && prev.shape() == t.shape() && prev.dtype() == t.dtype() &&
                !prev.sameData(t) && prev.data_->buffer_.size() >= t.numBytes()) {
                t.data_->buffer_ = std::move(prev.data_->buffer_);
            } else {
                t.bindBuffer(bufferPool_->requestBuffer(t.numBytes()));
            }
        }
        if (!t.data_->hostUploaded_) t.upload(stream());
        (*in)["out0"] = t;
    }
}

void NeuralNet::bindFusion()
{
    for (Node* n : sortedNodes_) {
        auto* lin = dynamic_cast<node::Linear*>(n);
        if (!lin) continue;
        lin->setFusedGate(nullptr);
        if (!config_.fuseGatedLinear) continue;
        NodeSlot& out = lin->slot("out0");
        if (out.connections().size() != 1) continue;
        auto* gm = dynamic_cast<node::GatedMul*>(&out.connections()[0]->parentNode());
        if (gm && lin->canFuseGate(*gm)) lin->setFusedGate(gm);
    }
}

void NeuralNet::recordCommands(const TensorRefDict& outputs)
{
    destroyGraph();
    bindFusion();
    scratch_.clear();
    // Propagate tensors along the wiring and let each node choose its kernel
    // and output shape; bind device buffers to outputs and temporaries.
    for (Node* n : sortedNodes_) {
        for (auto& [name, s] : n->slots_)
            if (s.type_ == NodeSlot::input && !s.connections_.empty()) s.value_ = s.connections_[0]->value_;
        if (n->kind() == std::string("Input")) continue;
        n->prepare();
        for (auto& [name, s] : n->slots_) {
            if (s.type_ != NodeSlot::output && s.type_ != NodeSlot::temporary) continue;
            Tensor& t = s.value_;
            if (!t.validShape()) continue;
            if (auto* lin = dynamic_cast<node::Linear*>(n); lin && lin->fusedGate() && name == "out0")
                continue;   // never materialised: the gated kernel writes GatedMul's output
            t.bindBuffer(bufferPool_->requestBuffer(t.numBytes()));
        }
    }
    for (auto& [name, out] : outputs_) {
        out.reached_ = out.slot("in0").getValueRef().validShape();
        out.cachedOutput_ = out.slot("in0").getValueRef();
    }
    for (InputNode* in : activeInputs_) {
        in->recordedShape_ = (*in)["in0"].shape();
        in->recordedPtr_ = (*in)["in0"].devicePtr();
    }
    CommandStream cmd(stream());
    if (config_.useGraph) {
        check(vai_graph_begin_capture((vai_stream_t)stream_), "graph capture");
        try {
            for (Node* n : sortedNodes_) n->run(cmd);
        } catch (...) {
            vai_graph_t g = nullptr;
            vai_graph_end_capture((vai_stream_t)stream_, &g);
            vai_graph_destroy(g);
            throw;
        }
        vai_graph_t g = nullptr;
        check(vai_graph_end_capture((vai_stream_t)stream_, &g), "graph end capture");
        graph_ = g;
    }
    ++recordCount_;
    (void)outputs;
}

void NeuralNet::launch()
{
    if (graph_) {
        check(vai_graph_launch((vai_graph_t)graph_, (vai_stream_t)stream_), "graph launch");
    } else {
        CommandStream cmd(stream_);
        for (Node* n : sortedNodes_) n->run(cmd);
    }
}

void NeuralNet::operator()(TensorDict inputs, TensorRefDict outputs, bool syncPrev)
{
    require(!inputs.empty(), "a forward needs at least one input");
    std::vector<InputNode*> active;
    for (auto& [name, tensor] : inputs) {
        auto it = inputs_.find(name);
        require(it != inputs_.end(), "no input named " + name);
        it->second["in0"] = tensor;
        active.push_back(&it->second);
    }
    if (active != activeInputs_) {
        activeInputs_ = std::move(active);
        needToRerecord_ = true;
    }
    if (syncPrev) sync();
    currentNet_ = this;
    if (needToRebuildGraph_) {
        sortNodes();
        needToRebuildGraph_ = false;
        needToUploadParams_ = true;
    }
    // A parameter set after the first forward (a new weight tensor on a
    // node) still has only host data: upload it and record again.
    if (!needToUploadParams_)
        for (Node* n : sortedNodes_)
            for (auto& [name, sl] : n->slots_)
                if (sl.type_ == NodeSlot::persistent && sl.value_.validShape() && sl.value_.hasHostData() &&
                    !sl.value_.gpuBufferBound())
                    needToUploadParams_ = true;
    if (needToUploadParams_) {
        uploadModelParams();
        needToUploadParams_ = false;
        needToRerecord_ = true;
    }
    prepareInputs();
    for (InputNode* in : activeInputs_)
        if (in->recordedShape_ != (*in)["in0"].shape() || in->recordedPtr_ != (*in)["in0"].devicePtr())
            needToRerecord_ = true;
    if (needToRerecord_) {
        recordCommands(outputs);
        needToRerecord_ = false;
    }
    launch();
    ++submitCount_;
    for (auto& [name, node] : outputs_)
        if (node.reached_) node.cachedOutput_.data_->lastSubmission_ = {this, submitCount_};
    for (auto& [name, dst] : outputs) {
        require(dst != nullptr, "null output tensor pointer");
        auto it = outputs_.find(name);
        require(it != outputs_.end(), "no output named " + name);
        *dst = it->second.reached_ ? it->second.cachedOutput_ : Tensor{};
    }
}

}   // namespace vai

// neural-net.h -- the graph API the MI355X kernels sit behind: Node, NodeSlot,
// NeuralNet with the reference's surface (/root/reference/vai/engine/
// neural-net.h:82-450). Differences, all below the API:
//  * a node records its launches on a vai::CommandStream (a HIP stream) in
//    run(); the reference records into an eva::CommandBuffer;
//  * NeuralNet records the forward once into a HIP graph and replays it while
//    the input shapes and buffers stay the same (the reference resubmits its
//    recorded command buffer, neural-net.h:377-449);
//  * a Linear whose only consumer is a GatedMul is fused with it at record
//    time (one MFMA kernel writes the gated output; the [M, 2H] intermediate
//    is never materialised).
// Gate branches and partial inputs (GraphController) are not part of this
// build.
#pragma once
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "tensor.h"

namespace vai {

class Node;
class NodeSlot;
class NeuralNet;
struct NodeFlow;

using TensorDict = std::map<std::string, Tensor>;
using TensorRefDict = std::map<std::string, Tensor*>;

// What a node records its launches on: a HIP stream, owned by the net.
class CommandStream
{
    void* stream_ = nullptr;

public:
    explicit CommandStream(void* s = nullptr) : stream_(s) {}
    void* stream() const { return stream_; }
};

class NodeSlot
{
    friend class NeuralNet;

public:
    enum Type { input, output, temporary, persistent, none };

private:
    Type type_;
    Node& parent_;
    std::vector<NodeSlot*> connections_;
    Tensor value_;

public:
    NodeSlot(Type type, Node* parent) : type_(type), parent_(*parent) {}
    Type type() const { return type_; }
    const Node& parent() const { return parent_; }
    Node& parentNode() { return parent_; }
    const std::vector<NodeSlot*>& connections() const { return connections_; }
    Tensor& getValueRef() { return value_; }
    const Tensor& getValueRef() const { return value_; }

    // /root/reference/vai/engine/neural-net.h:124-131 (an input takes one producer).
    static void connect(NodeSlot& a, NodeSlot& b);
    static void disconnect(NodeSlot& a, NodeSlot& b);
};

// Only NeuralNet makes one (NeuralNet::dtypeKey()), so the nodes' dtype
// setters are a model net's to call (neural-net.h:134-141).
class DtypeKey
{
    friend class NeuralNet;
    DtypeKey() = default;
};

class Node
{
    friend class NeuralNet;
    std::map<std::string, NodeSlot> slots_;

protected:
    NeuralNet* ownedNet_ = nullptr;
    Dtype oDtype_ = Dtype::None;
    void addSlot(const std::string& name, NodeSlot::Type type) { slots_.try_emplace(name, type, this); }
    // The dtype this node writes: setODtype's, else the net's default.
    Dtype outputDtype() const;

public:
    Node();
    virtual ~Node() = default;

    Dtype wDefaultDtype() const;
    Dtype oDefaultDtype() const;
    BufferPool& bufferPool() const;
    NeuralNet& net() const { return *ownedNet_; }
    void setODtype(Dtype dtype, DtypeKey) { oDtype_ = dtype; }

    const std::map<std::string, NodeSlot>& slots() const { return slots_; }
    NodeSlot& slot(const std::string& name);
    const NodeSlot* findSlot(const std::string& name) const
    {
        auto it = slots_.find(name);
        return it == slots_.end() ? nullptr : &it->second;
    }
    Tensor& operator[](const std::string& name) { return slot(name).getValueRef(); }
    const Tensor& operator[](const std::string& name) const { return slots_.at(name).getValueRef(); }

    operator NodeFlow();

    // Validate inputs, choose the kernel, set output shapes (no launches).
    virtual void prepare() = 0;
    // Launch this node's kernels on cmd.
    virtual void run(CommandStream& cmd) = 0;
    // Device scratch the node needs during run(), bound to its "temporary"
    // slots by the net before run(); 0 when none.
    virtual size_t workspaceBytes() const { return 0; }
    // Kind tag for record-time fusion ("Linear", "GatedMul", ...).
    virtual const char* kind() const { return "Node"; }
};

class InputNode : public Node
{
    friend class NeuralNet;
    std::vector<uint32_t> recordedShape_;
    void* recordedPtr_ = nullptr;

public:
    InputNode();
    void prepare() override {}
    void run(CommandStream&) override {}
    const char* kind() const override { return "Input"; }
};

class OutputNode : public Node
{
    friend class NeuralNet;
    Tensor cachedOutput_;
    bool reached_ = false;

public:
    OutputNode();
    void prepare() override;
    void run(CommandStream&) override {}
    const char* kind() const override { return "Output"; }
};

// /root/reference/vai/engine/neural-net.h:261-284.
struct NeuralNetConfig
{
    int device = 0;
    size_t uploadChunkSizeMiB = 256;
    std::shared_ptr<BufferPool> bufferPool = nullptr;
    uint32_t bufferPoolLogLevel = 0;
    Dtype wDefaultDtype = Dtype::Fp16;
    Dtype oDefaultDtype = Dtype::Fp32;
    bool useGraph = true;          // record the forward into a HIP graph and replay it
    bool fuseGatedLinear = true;   // Linear -> GatedMul becomes one gated GEMM
};

class NeuralNet
{
    friend class Node;
    friend class InputNode;
    friend class OutputNode;

    thread_local inline static NeuralNet* currentNet_ = nullptr;

    NeuralNetConfig config_;
    std::shared_ptr<BufferPool> bufferPool_;
    void* stream_ = nullptr;
    void* graph_ = nullptr;

    std::vector<Node*> sortedNodes_;
    std::map<std::string, InputNode> inputs_;
    std::map<std::string, OutputNode> outputs_;
    std::vector<InputNode*> activeInputs_;
    std::vector<PooledBuffer> scratch_;

    bool needToRebuildGraph_ = true;
    bool needToUploadParams_ = true;
    bool needToRerecord_ = true;
    uint64_t submitCount_ = 0;
    uint64_t recordCount_ = 0;

    void destroyGraph();
    void launch();
    void bindFusion();

protected:
    static DtypeKey dtypeKey() { return {}; }

public:
    static NeuralNet* current() { return currentNet_; }

    explicit NeuralNet(const NeuralNetConfig& config = {});
    virtual ~NeuralNet();
    NeuralNet(const NeuralNet&) = delete;
    NeuralNet& operator=(const NeuralNet&) = delete;

    const NeuralNetConfig& config() const { return config_; }
    BufferPool& bufferPool() const { return *bufferPool_; }
    std::shared_ptr<BufferPool> bufferPoolPtr() const { return bufferPool_; }
    void* stream();   // the net's HIP stream, created on first use

    InputNode& input(const std::string& name) { return inputs_.try_emplace(name).first->second; }
    OutputNode& output(const std::string& name) { return outputs_.try_emplace(name).first->second; }

    void invalidateCommandBuffer() { needToRerecord_ = true; }
    // Wait for the last submitted forward.
    void sync();
    // Kahn's algorithm over the wiring (neural-net.cpp:282-354); throws on a
    // cycle or on an input slot with more than one producer.
    void sortNodes();
    void uploadModelParams();
    void prepareInputs();
    void recordCommands(const TensorRefDict& outputs);

    // How many times the forward was recorded (a replay does not record).
    uint64_t recordCount() const { return recordCount_; }
    uint64_t submitCount() const { return submitCount_; }
    const std::vector<Node*>& sortedNodes() const { return sortedNodes_; }
    std::vector<std::string> outputNames() const
    {
        std::vector<std::string> v;
        for (const auto& [name, node] : outputs_) v.push_back(name);
        return v;
    }

    void operator()(TensorDict inputs, TensorRefDict outputs, bool syncPrev = true);
};

}   // namespace vai

// graph-flow.h -- the wiring DSL of the reference (/root/reference/vai/engine/
// graph-flow.h:13-141): `a - b` connects a's output slot to b's input slot and
// yields b, `"name"/node` picks an input slot, `node/"name"` an output slot;
// unnamed sides are in0 / out0. NodeGroup republishes member slots so a
// subgraph wires like one node. The operators are the API, so they keep the
// reference's spelling and meaning.
#pragma once
#include <string>
#include <utility>

#include "neural-net.h"

namespace vai {

struct NodeFlow
{
    std::string inSlotName;
    Node& node;
    std::string outSlotName;
};

inline Node::operator NodeFlow() { return NodeFlow{"in0", *this, "out0"}; }
inline NodeFlow operator/(std::string name, Node& node) { return {std::move(name), node, "out0"}; }
inline NodeFlow operator/(Node& node, std::string name) { return {"in0", node, std::move(name)}; }
inline NodeFlow&& operator/(NodeFlow&& f, std::string name)
{
    f.outSlotName = std::move(name);
    return std::move(f);
}

inline void operator-(NodeSlot& a, NodeSlot& b) { NodeSlot::connect(a, b); }

inline NodeFlow&& operator-(NodeFlow&& in, NodeFlow&& out)
{
    in.node.slot(in.outSlotName) - out.node.slot(out.inSlotName);
    return std::move(out);
}

struct GroupFlow;

class NodeGroup
{
    std::map<std::string, NodeSlot*> slots_;

protected:
    NeuralNet* ownedNet_ = nullptr;
    void defineSlot(const std::string& name, NodeSlot& slot) { slots_.try_emplace(name, &slot); }

public:
    NodeGroup() : ownedNet_(NeuralNet::current()) {}
    virtual ~NodeGroup() = default;
    NodeSlot& slot(const std::string& name)
    {
        auto it = slots_.find(name);
        require(it != slots_.end(), "NodeGroup: no slot named " + name);
        return *it->second;
    }
    operator GroupFlow();
};

struct GroupFlow
{
    std::string inSlotName;
    NodeGroup& group;
    std::string outSlotName;
};

inline NodeGroup::operator GroupFlow() { return {"in0", *this, "out0"}; }
inline GroupFlow operator/(std::string name, NodeGroup& g) { return {std::move(name), g, "out0"}; }
inline GroupFlow operator/(NodeGroup& g, std::string name) { return {"in0", g, std::move(name)}; }
inline GroupFlow&& operator/(GroupFlow&& f, std::string name)
{
    f.outSlotName = std::move(name);
    return std::move(f);
}
inline GroupFlow&& operator-(GroupFlow&& in, GroupFlow&& out)
{
    in.group.slot(in.outSlotName) - out.group.slot(out.inSlotName);
    return std::move(out);
}
inline GroupFlow&& operator-(NodeFlow&& in, GroupFlow&& out)
{
    in.node.slot(in.outSlotName) - out.group.slot(out.inSlotName);
    return std::move(out);
}
inline NodeFlow&& operator-(GroupFlow&& in, NodeFlow&& out)
{
    in.group.slot(in.outSlotName) - out.node.slot(out.inSlotName);
    return std::move(out);
}

}   // namespace vai

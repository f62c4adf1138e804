// Strict JSON parser with explicit limits, in the manner of src/json/mod.rs:
// RFC 8259 objects, arrays, numbers, strings and escapes; duplicate keys,
// trailing commas, leading zeros, unescaped control characters, lone
// surrogates, non-finite numbers and trailing content are rejected (CORRUPT);
// the input size, nesting depth, string length, container entries and total
// value count are capped (LIMIT).
//
// The document is a flat tape: nodes in pre-order, each container node
// followed by its children (an object's members as key node, value subtree),
// and every node records the index just past its subtree. Strings are
// unescaped into one arena reserved to the input size, so views into it stay
// valid for the life of the document.
#pragma once

#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

#include "../../include/svl_hip.h"

namespace svl::json {

enum class Type : uint8_t { Null, Bool, UInt, Int, Float, String, Array, Object };

struct Node {
    Type type;
    bool b;
    uint32_t count;  // array elements / object members
    uint32_t next;   // index just past this node's subtree
    uint32_t off, len;  // string bytes in the arena
    union {
        uint64_t u;
        int64_t i;
        double f;
    };
};

struct Limits {
    size_t max_input_bytes;
    size_t max_depth;
    size_t max_string_bytes;
    size_t max_container_entries;
    size_t max_total_values;
};

class Doc {
public:
    std::vector<Node> nodes;
    std::string arena;

    const Node &at(uint32_t i) const { return nodes[i]; }
    Type type(uint32_t i) const { return nodes[i].type; }
    std::string_view str(uint32_t i) const {
        return std::string_view(arena.data() + nodes[i].off, nodes[i].len);
    }
    // Member `key` of object node i, or UINT32_MAX.
    uint32_t get(uint32_t i, std::string_view key) const;
    // Children of array node i / members (key index) of object node i.
    template <class F>
    void each(uint32_t i, F &&f) const {
        uint32_t k = i + 1;
        for (uint32_t n = 0; n < nodes[i].count; ++n) {
            if (nodes[i].type == Type::Object) {
                f(k, k + 1);
                k = nodes[k + 1].next;
            } else {
                f(k, k);
                k = nodes[k].next;
            }
        }
    }
    // Exact non-negative integer value (Number::as_u64, json/mod.rs:50-56).
    bool as_u64(uint32_t i, uint64_t &out) const;
};

// Parses `len` bytes of UTF-8 text. On failure returns CORRUPT or LIMIT with
// the message in `err`.
svl_status parse(const char *text, size_t len, const Limits &limits, Doc &doc, std::string &err);

// Whether `len` bytes are well-formed UTF-8 (no surrogates, no overlongs).
bool valid_utf8(const char *text, size_t len);

}  // namespace svl::json

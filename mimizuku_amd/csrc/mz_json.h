// Strict JSON (RFC 8259) for safetensors headers and the model directory's configs, host side.
// Follows src/json.rs: at most 64 levels of nesting, finite numbers in the RFC grammar only, no control characters in
// strings, \u escapes with surrogate pairs (an unpaired surrogate becomes U+FFFD and what follows it is kept), the
// text of every string valid UTF-8, nothing but whitespace after the value. Object members keep their order and
// duplicates (lookups return the first).
#pragma once
#include <stddef.h>

#include <string>
#include <utility>
#include <vector>

struct MzJson {
    enum Kind { OBJ, ARR, STR, NUM, BOOL, NUL } kind = NUL;
    std::vector<std::pair<std::string, MzJson>> obj;
    std::vector<MzJson> arr;
    std::string str;
    double num = 0.0;
    bool b = false;

    const MzJson* get(const char* key) const;  // first member named key of an object, else null
    // a non-negative integer that a double represents exactly (json.rs:30-32)
    bool uint(size_t* out) const;
    // an array of such integers; false if any entry is not one
    bool uints(std::vector<size_t>* out) const;
};

// Parses s[0 .. n). On failure returns false and sets *err to a message that names the byte offset.
bool mz_json_parse(const char* s, size_t n, MzJson* out, std::string* err);

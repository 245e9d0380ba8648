// types.cpp -- the ggml type table of g4run.h:80-94 with its block geometry
// (gguf.c:11-25) and the row sizes derived from it (g4run.h:95-99).  Host
// code only, so the GGUF parser builds with it alone (its sanitizer test).
#include "../../include/g4run_abi.h"

#include "../../include/g4hip.h"

namespace {
struct TypeRow {
    int t;
    const char *name;
    int blck, size;
};
const TypeRow kTypes[] = {
    {G4H_F32, "F32", 1, 4},       {G4H_F16, "F16", 1, 2},        {G4H_BF16, "BF16", 1, 2},
    {G4H_Q4_0, "Q4_0", 32, 18},   {G4H_Q8_0, "Q8_0", 32, 34},    {G4H_Q2_K, "Q2_K", 256, 84},
    {G4H_Q3_K, "Q3_K", 256, 110}, {G4H_Q4_K, "Q4_K", 256, 144},  {G4H_Q5_K, "Q5_K", 256, 176},
    {G4H_Q6_K, "Q6_K", 256, 210}, {G4H_TQ2_0, "TQ2_0", 256, 66}, {24, "I8", 1, 1},
    {25, "I16", 1, 2},            {26, "I32", 1, 4},             {27, "I64", 1, 8},
    {28, "F64", 1, 8},
};
const TypeRow *find_type(int t) {
    for (const TypeRow &r : kTypes)
        if (r.t == t) return &r;
    return nullptr;
}
}  // namespace

extern "C" const char *g4_type_name(int t) { const TypeRow *r = find_type(t); return r ? r->name : "?"; }
extern "C" int g4_type_blck(int t) { const TypeRow *r = find_type(t); return r ? r->blck : 0; }
extern "C" size_t g4_type_size(int t) { const TypeRow *r = find_type(t); return r ? (size_t)r->size : 0; }
extern "C" size_t g4_row_size(int t, int64_t n) {
    const int b = g4_type_blck(t);
    if (!b || n % b) return 0;
    return (size_t)(n / b) * g4_type_size(t);
}

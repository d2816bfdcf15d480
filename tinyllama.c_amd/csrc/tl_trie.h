/*
 * tl_trie.h — token trie: a map from token strings (u32 sequences) to a
 * non-zero u32 value.
 *
 * It provides what the KV prefix cache needs from the reference's radix tree
 * (src/rax.c, used by src/kvcache.c as "token prefix -> slot + 1"): find,
 * insert and remove of whole keys.  Keys are u32 token strings instead of
 * byte strings; every key the KV cache stores is a whole number of tokens,
 * so the two maps hold the same keys and answer the same lookups.
 *
 * Layout: one node per stored prefix; edges live in one open-addressing
 * hash table keyed by (parent node, token), so walking one token is one
 * hash probe and a walk can resume from any node (the KV cache keeps a
 * cursor at the end of the current request's prefix).
 */
#ifndef TL_TRIE_H
#define TL_TRIE_H

#include <stdbool.h>
#include <stdint.h>

#define TL_TRIE_NONE  UINT32_MAX
#define TL_TRIE_ROOT  0u

typedef struct {
    uint32_t parent;    /* TL_TRIE_NONE for the root */
    uint32_t token;
    uint32_t value;     /* 0 = no key ends here */
    uint32_t n_child;
} TlTrieNode;

typedef struct {
    TlTrieNode *nodes;
    uint32_t    n_nodes;     /* high-water mark of node ids */
    uint32_t    cap_nodes;
    uint32_t   *free_ids;    /* recycled node ids */
    uint32_t    n_free;
    uint64_t   *hkey;        /* (parent << 32) | token, or TL_TRIE_EMPTY */
    uint32_t   *hval;        /* child node id */
    uint32_t    hmask;       /* table size - 1 (power of two) */
    uint32_t    hcount;
    uint64_t    epoch;       /* bumped whenever a node is freed */
} TlTrie;

bool     tl_trie_init(TlTrie *t, uint32_t expect_nodes);
void     tl_trie_free(TlTrie *t);
/* child of `node` along `token`, or TL_TRIE_NONE */
uint32_t tl_trie_child(const TlTrie *t, uint32_t node, uint32_t token);
/* child of `node` along `token`, created when missing; TL_TRIE_NONE on OOM */
uint32_t tl_trie_child_make(TlTrie *t, uint32_t node, uint32_t token);
/* node reached by `key[0..len)` from `from`, or TL_TRIE_NONE */
uint32_t tl_trie_walk(const TlTrie *t, uint32_t from, const uint32_t *key, uint32_t len);
/* clear the value stored at key[0..len) and free nodes that no longer lead
 * to any key; no-op when the key is absent */
void     tl_trie_remove(TlTrie *t, const uint32_t *key, uint32_t len);
/* the same for the key that ends at node `n` (a node id returned by
 * tl_trie_child / tl_trie_child_make whose value is set) */
void     tl_trie_remove_node(TlTrie *t, uint32_t n);
/* number of keys currently stored (nodes with a value) */
uint32_t tl_trie_count(const TlTrie *t);

#endif

/* tl_trie.c — token trie with a single (parent, token) -> child hash table. */
#include "tl_trie.h"

#include <stdlib.h>
#include <string.h>

#define TL_TRIE_EMPTY UINT64_MAX

static inline uint64_t edge_key(uint32_t parent, uint32_t token) {
    return ((uint64_t)parent << 32) | token;
}

static inline uint32_t edge_hash(uint64_t k) {
    /* splitmix64 finaliser */
    k ^= k >> 30;
    k *= 0xbf58476d1ce4e5b9ull;
    k ^= k >> 27;
    k *= 0x94d049bb133111ebull;
    k ^= k >> 31;
    return (uint32_t)k;
}

static bool table_alloc(TlTrie *t, uint32_t size) {
    t->hkey = (uint64_t *)malloc((size_t)size * sizeof(uint64_t));
    t->hval = (uint32_t *)malloc((size_t)size * sizeof(uint32_t));
    if (!t->hkey || !t->hval) {
        free(t->hkey);
        free(t->hval);
        t->hkey = NULL;
        t->hval = NULL;
        return false;
    }
    for (uint32_t i = 0; i < size; i++) t->hkey[i] = TL_TRIE_EMPTY;
    t->hmask = size - 1;
    t->hcount = 0;
    return true;
}

static void table_put(TlTrie *t, uint64_t k, uint32_t v) {
    uint32_t i = edge_hash(k) & t->hmask;
    while (t->hkey[i] != TL_TRIE_EMPTY) i = (i + 1) & t->hmask;
    t->hkey[i] = k;
    t->hval[i] = v;
    t->hcount++;
}

static bool table_grow(TlTrie *t) {
    uint64_t *ok = t->hkey;
    uint32_t *ov = t->hval;
    uint32_t osize = t->hmask + 1;
    if (!table_alloc(t, osize * 2)) {
        t->hkey = ok;
        t->hval = ov;
        t->hmask = osize - 1;
        return false;
    }
    for (uint32_t i = 0; i < osize; i++)
        if (ok[i] != TL_TRIE_EMPTY) table_put(t, ok[i], ov[i]);
    free(ok);
    free(ov);
    return true;
}

/* linear-probing delete with backward shift (no tombstones) */
static void table_del(TlTrie *t, uint64_t k) {
    uint32_t i = edge_hash(k) & t->hmask;
    while (t->hkey[i] != k) {
        if (t->hkey[i] == TL_TRIE_EMPTY) return;
        i = (i + 1) & t->hmask;
    }
    uint32_t j = i;
    for (;;) {
        j = (j + 1) & t->hmask;
        if (t->hkey[j] == TL_TRIE_EMPTY) break;
        uint32_t home = edge_hash(t->hkey[j]) & t->hmask;
        /* move j back to i when its home is not cyclically in (i, j] */
        bool in_range = (i <= j) ? (home > i && home <= j) : (home > i || home <= j);
        if (!in_range) {
            t->hkey[i] = t->hkey[j];
            t->hval[i] = t->hval[j];
            i = j;
        }
    }
    t->hkey[i] = TL_TRIE_EMPTY;
    t->hcount--;
}

bool tl_trie_init(TlTrie *t, uint32_t expect_nodes) {
    memset(t, 0, sizeof(*t));
    uint32_t cap = expect_nodes < 64 ? 64 : expect_nodes + 1;
    uint32_t hsize = 128;
    while (hsize < 2 * cap) hsize <<= 1;
    t->nodes = (TlTrieNode *)malloc((size_t)cap * sizeof(TlTrieNode));
    t->free_ids = (uint32_t *)malloc((size_t)cap * sizeof(uint32_t));
    if (!t->nodes || !t->free_ids || !table_alloc(t, hsize)) {
        tl_trie_free(t);
        return false;
    }
    t->cap_nodes = cap;
    t->nodes[TL_TRIE_ROOT] = (TlTrieNode){TL_TRIE_NONE, 0, 0, 0};
    t->n_nodes = 1;
    return true;
}

void tl_trie_free(TlTrie *t) {
    if (!t) return;
    free(t->nodes);
    free(t->free_ids);
    free(t->hkey);
    free(t->hval);
    memset(t, 0, sizeof(*t));
}

uint32_t tl_trie_child(const TlTrie *t, uint32_t node, uint32_t token) {
    if (node == TL_TRIE_NONE) return TL_TRIE_NONE;
    uint64_t k = edge_key(node, token);
    uint32_t i = edge_hash(k) & t->hmask;
    for (;;) {
        uint64_t h = t->hkey[i];
        if (h == k) return t->hval[i];
        if (h == TL_TRIE_EMPTY) return TL_TRIE_NONE;
        i = (i + 1) & t->hmask;
    }
}

static uint32_t node_alloc(TlTrie *t) {
    if (t->n_free) return t->free_ids[--t->n_free];
    if (t->n_nodes == t->cap_nodes) {
        uint32_t ncap = t->cap_nodes * 2;
        TlTrieNode *nn = (TlTrieNode *)realloc(t->nodes, (size_t)ncap * sizeof(TlTrieNode));
        if (!nn) return TL_TRIE_NONE;
        t->nodes = nn;
        uint32_t *nf = (uint32_t *)realloc(t->free_ids, (size_t)ncap * sizeof(uint32_t));
        if (!nf) return TL_TRIE_NONE;
        t->free_ids = nf;
        t->cap_nodes = ncap;
    }
    return t->n_nodes++;
}

uint32_t tl_trie_child_make(TlTrie *t, uint32_t node, uint32_t token) {
    uint32_t c = tl_trie_child(t, node, token);
    if (c != TL_TRIE_NONE || node == TL_TRIE_NONE) return c;
    if ((t->hcount + 1) * 2 > t->hmask + 1 && !table_grow(t)) return TL_TRIE_NONE;
    c = node_alloc(t);
    if (c == TL_TRIE_NONE) return c;
    t->nodes[c] = (TlTrieNode){node, token, 0, 0};
    t->nodes[node].n_child++;
    table_put(t, edge_key(node, token), c);
    return c;
}

uint32_t tl_trie_walk(const TlTrie *t, uint32_t from, const uint32_t *key, uint32_t len) {
    uint32_t n = from;
    for (uint32_t i = 0; i < len && n != TL_TRIE_NONE; i++) n = tl_trie_child(t, n, key[i]);
    return n;
}

void tl_trie_remove(TlTrie *t, const uint32_t *key, uint32_t len) {
    tl_trie_remove_node(t, tl_trie_walk(t, TL_TRIE_ROOT, key, len));
}

void tl_trie_remove_node(TlTrie *t, uint32_t n) {
    if (n == TL_TRIE_NONE || n == TL_TRIE_ROOT || n >= t->n_nodes || t->nodes[n].value == 0) return;
    t->nodes[n].value = 0;
    /* prune: a node with no value and no children leads to no key */
    while (n != TL_TRIE_ROOT && t->nodes[n].value == 0 && t->nodes[n].n_child == 0) {
        uint32_t parent = t->nodes[n].parent;
        table_del(t, edge_key(parent, t->nodes[n].token));
        t->nodes[parent].n_child--;
        t->free_ids[t->n_free++] = n;
        t->epoch++;
        n = parent;
    }
}

uint32_t tl_trie_count(const TlTrie *t) {
    uint32_t c = 0;
    /* free ids are marked by walking the free list once */
    uint8_t *dead = (uint8_t *)calloc(t->n_nodes ? t->n_nodes : 1, 1);
    if (!dead) return 0;
    for (uint32_t i = 0; i < t->n_free; i++) dead[t->free_ids[i]] = 1;
    for (uint32_t i = 1; i < t->n_nodes; i++)
        if (!dead[i] && t->nodes[i].value) c++;
    free(dead);
    return c;
}

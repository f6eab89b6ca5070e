// batcher.cpp -- host-side continuous batching over the paged KV pool.
//
// The bookkeeping of the reference scheduler (src/continuous_batch.cu:48-174,
// include/scheduler.h:6-54) on top of the LIFO block allocator of
// src/paged_kvcache.cu:49-53,89-98, rebuilt so that one step serves every
// active sequence with ONE batched forward instead of one forward per
// sequence: each plan lists, per sequence in active order, its query rows
// (the whole prompt for a prefill, the newest token for a decode) with their
// token ids, positions and KV slots, its context length and its block table --
// exactly the arrays ql_rope_paged_kv_append_f16 / ql_paged_kv_append_f16
// (slot_mapping) and ql_paged_attention_f16 (cu_q_lens, ctx_lens,
// block_tables) take.
//
// Rules kept from the reference:
//   admission   FIFO; the head request is admitted when fewer than max_active
//               sequences run and ceil(prompt_len/16) blocks are free (they are
//               taken at once); otherwise admission stops for this step
//               (head-of-line blocking) (continuous_batch.cu:71-87).
//   growth      a decoding sequence whose next position starts a new 16-token
//               block takes one more block before its step; with none free it
//               is evicted (finished early, no work this step) (:113-121).
//   finishing   when the sequence reaches prompt_len + max_gen tokens or
//               samples the end-of-sequence token (2 in the reference) (:136-138).
//   ejection    finished sequences return their blocks in table order and leave
//               the active list by swap-with-last, which reorders it (:141-168).
// Difference: the reference discards the token sampled after the prefill (its
// forward is a stub); here it is the first generated token, so a sequence
// reaches prompt_len + max_gen tokens one step earlier.  Block growth and
// eviction happen at the same token positions as in the reference.
#include "quantlib_amd.h"

#include <algorithm>
#include <deque>
#include <new>
#include <vector>

#define QL_CHECK_BATCHER(cond)                     \
    do {                                           \
        if (!(cond)) return hipErrorInvalidValue;  \
    } while (0)

namespace {

enum class State { kPending, kPrefill, kDecode, kFinished };

struct Seq {
    int req_id = 0;
    std::vector<int32_t> tokens;   // prompt then generated tokens
    int prompt_len = 0;
    int max_tokens = 0;            // prompt_len + max_gen
    State state = State::kPending;
    int reason = QL_FINISH_LENGTH;
    std::vector<int32_t> blocks;   // logical -> physical block
    int seq_len() const { return (int)tokens.size(); }
};

struct Finished {
    int req_id, reason, prompt_len;
    std::vector<int32_t> tokens;
};

}  // namespace

struct ql_batcher {
    // allocator: LIFO stack of free block indices, owned or borrowed
    std::vector<int> own_stack;
    int* stack = nullptr;
    int* free_count = nullptr;
    int own_count = 0;
    int n_blocks = 0;
    int max_active = 0;
    int eos = 2;
    std::deque<Seq*> pending;
    std::vector<Seq*> active;
    std::deque<Finished> finished;
    // plan
    bool planned = false;
    std::vector<Seq*> plan_seqs;
    std::vector<int32_t> req_ids, is_prefill, cu_q, ctx, tables, tok, pos, slot, sample_rows;

    int take_block() {   // paged_kv_allocate_block
        if (*free_count == 0) return -1;
        --*free_count;
        return stack[*free_count];
    }
    void give_block(int b) {   // paged_kv_free_block
        if (b < 0 || b >= n_blocks || *free_count >= n_blocks) return;
        stack[*free_count] = b;
        ++*free_count;
    }
};

namespace {

hipError_t make(ql_batcher* b, int n_blocks, int max_active, int eos_token, ql_batcher** out) {
    b->n_blocks = n_blocks;
    b->max_active = max_active;
    b->eos = eos_token;
    *out = b;
    return hipSuccess;
}

void finish(ql_batcher* b, Seq* s) {
    for (int blk : s->blocks) b->give_block(blk);
    s->blocks.clear();
    b->finished.push_back(Finished{s->req_id, s->reason, s->prompt_len, std::move(s->tokens)});
    delete s;
}

}  // namespace

extern "C" hipError_t ql_batcher_create(int n_blocks, int max_active, int eos_token,
                                        ql_batcher** out) {
    QL_CHECK_BATCHER(out && n_blocks >= 0 && max_active > 0);
    ql_batcher* b = new (std::nothrow) ql_batcher();
    if (!b) return hipErrorOutOfMemory;
    b->own_stack.resize((size_t)n_blocks);
    for (int i = 0; i < n_blocks; ++i) b->own_stack[(size_t)i] = n_blocks - 1 - i;   // pops 0, 1, 2, ...
    b->own_count = n_blocks;
    b->stack = b->own_stack.data();
    b->free_count = &b->own_count;
    return make(b, n_blocks, max_active, eos_token, out);
}

extern "C" hipError_t ql_batcher_create_on_stack(int* free_blocks, int* free_count, int n_blocks,
                                                 int max_active, int eos_token, ql_batcher** out) {
    QL_CHECK_BATCHER(out && free_blocks && free_count && n_blocks >= 0 && max_active > 0);
    QL_CHECK_BATCHER(*free_count >= 0 && *free_count <= n_blocks);
    ql_batcher* b = new (std::nothrow) ql_batcher();
    if (!b) return hipErrorOutOfMemory;
    b->stack = free_blocks;
    b->free_count = free_count;
    return make(b, n_blocks, max_active, eos_token, out);
}

extern "C" hipError_t ql_batcher_destroy(ql_batcher* b) {
    if (!b) return hipSuccess;
    for (Seq* s : b->active) {
        for (int blk : s->blocks) b->give_block(blk);
        delete s;
    }
    for (Seq* s : b->pending) delete s;
    delete b;
    return hipSuccess;
}

extern "C" hipError_t ql_batcher_add_request(ql_batcher* b, int req_id, const int32_t* prompt,
                                             int prompt_len, int max_gen) {
    QL_CHECK_BATCHER(b && prompt && prompt_len > 0 && max_gen > 0);
    QL_CHECK_BATCHER((long long)prompt_len + max_gen <= (1LL << 30));
    Seq* s = new (std::nothrow) Seq();
    if (!s) return hipErrorOutOfMemory;
    s->req_id = req_id;
    s->prompt_len = prompt_len;
    s->max_tokens = prompt_len + max_gen;
    s->tokens.reserve((size_t)s->max_tokens);
    s->tokens.assign(prompt, prompt + prompt_len);
    b->pending.push_back(s);
    return hipSuccess;
}

extern "C" hipError_t ql_batcher_plan(ql_batcher* b, ql_step_plan* plan) {
    QL_CHECK_BATCHER(b && plan && !b->planned);
    constexpr int P = QL_PAGE_SIZE;
    // 1. admission (FIFO, head-of-line blocking)
    while (!b->pending.empty() && (int)b->active.size() < b->max_active) {
        Seq* s = b->pending.front();
        const int need = (s->prompt_len + P - 1) / P;
        if (*b->free_count < need) break;
        for (int i = 0; i < need; ++i) s->blocks.push_back(b->take_block());
        s->state = State::kPrefill;
        b->active.push_back(s);
        b->pending.pop_front();
    }
    // 2. growth / eviction, then the rows of every sequence that runs
    b->plan_seqs.clear();
    b->req_ids.clear();
    b->is_prefill.clear();
    b->cu_q.assign(1, 0);
    b->ctx.clear();
    b->tok.clear();
    b->pos.clear();
    b->slot.clear();
    b->sample_rows.clear();
    for (Seq* s : b->active) {
        int first, last;   // positions [first, last] run this step
        if (s->state == State::kPrefill) {
            first = 0;
            last = s->prompt_len - 1;
        } else if (s->state == State::kDecode) {
            first = last = s->seq_len() - 1;
            if (last / P >= (int)s->blocks.size()) {
                const int blk = b->take_block();
                if (blk < 0) {   // out of blocks: evicted, finished early
                    s->state = State::kFinished;
                    s->reason = QL_FINISH_EVICTED;
                    continue;
                }
                s->blocks.push_back(blk);
            }
        } else {
            continue;
        }
        b->plan_seqs.push_back(s);
        b->req_ids.push_back(s->req_id);
        b->is_prefill.push_back(s->state == State::kPrefill);
        for (int p = first; p <= last; ++p) {
            b->tok.push_back(s->tokens[(size_t)p]);
            b->pos.push_back(p);
            b->slot.push_back(s->blocks[(size_t)(p / P)] * P + p % P);
        }
        b->cu_q.push_back((int32_t)b->tok.size());
        b->ctx.push_back(last + 1);
        b->sample_rows.push_back((int32_t)b->tok.size() - 1);
    }
    const int n = (int)b->plan_seqs.size();
    int max_blocks = 0, max_q = 0, max_ctx = 0;
    for (int i = 0; i < n; ++i) {
        max_blocks = std::max(max_blocks, (int)b->plan_seqs[(size_t)i]->blocks.size());
        max_q = std::max(max_q, b->cu_q[(size_t)i + 1] - b->cu_q[(size_t)i]);
        max_ctx = std::max(max_ctx, (int)b->ctx[(size_t)i]);
    }
    b->tables.assign((size_t)n * (size_t)max_blocks, -1);
    for (int i = 0; i < n; ++i) {
        const std::vector<int32_t>& bl = b->plan_seqs[(size_t)i]->blocks;
        std::copy(bl.begin(), bl.end(), b->tables.begin() + (size_t)i * max_blocks);
    }
    plan->n_seqs = n;
    plan->n_rows = (int)b->tok.size();
    plan->max_q_len = max_q;
    plan->max_ctx_len = max_ctx;
    plan->max_blocks = max_blocks;
    plan->req_ids = b->req_ids.data();
    plan->is_prefill = b->is_prefill.data();
    plan->cu_q_lens = b->cu_q.data();
    plan->ctx_lens = b->ctx.data();
    plan->block_tables = b->tables.data();
    plan->token_ids = b->tok.data();
    plan->positions = b->pos.data();
    plan->slot_mapping = b->slot.data();
    plan->sample_rows = b->sample_rows.data();
    b->planned = true;
    return hipSuccess;
}

extern "C" hipError_t ql_batcher_commit(ql_batcher* b, const int32_t* sampled, int n_seqs) {
    QL_CHECK_BATCHER(b && b->planned && n_seqs == (int)b->plan_seqs.size());
    QL_CHECK_BATCHER(n_seqs == 0 || sampled);
    for (int i = 0; i < n_seqs; ++i) {
        Seq* s = b->plan_seqs[(size_t)i];
        const int32_t t = sampled[i];
        s->tokens.push_back(t);
        s->state = State::kDecode;
        if (t == b->eos) {
            s->state = State::kFinished;
            s->reason = QL_FINISH_EOS;
        } else if (s->seq_len() >= s->max_tokens) {
            s->state = State::kFinished;
            s->reason = QL_FINISH_LENGTH;
        }
    }
    // ejection: blocks back in table order, swap-with-last removal
    for (size_t i = 0; i < b->active.size();) {
        Seq* s = b->active[i];
        if (s->state == State::kFinished) {
            b->active[i] = b->active.back();
            b->active.pop_back();
            finish(b, s);
        } else {
            ++i;
        }
    }
    b->plan_seqs.clear();
    b->planned = false;
    return hipSuccess;
}

extern "C" hipError_t ql_batcher_stats(const ql_batcher* b, ql_batcher_counts* st) {
    QL_CHECK_BATCHER(b && st);
    st->n_active = (int)b->active.size();
    st->n_pending = (int)b->pending.size();
    st->free_blocks = *b->free_count;
    st->n_finished = (int)b->finished.size();
    return hipSuccess;
}

extern "C" hipError_t ql_batcher_pop_finished(ql_batcher* b, ql_finished* ev, int32_t* tokens,
                                              int cap, int* got) {
    QL_CHECK_BATCHER(b && ev && got && cap >= 0 && (cap == 0 || tokens));
    *got = 0;
    if (b->finished.empty()) return hipSuccess;
    Finished& f = b->finished.front();
    ev->req_id = f.req_id;
    ev->reason = f.reason;
    ev->prompt_len = f.prompt_len;
    ev->n_tokens = (int)f.tokens.size();
    const int n = std::min(cap, ev->n_tokens);
    std::copy(f.tokens.begin(), f.tokens.begin() + n, tokens);
    b->finished.pop_front();
    *got = 1;
    return hipSuccess;
}

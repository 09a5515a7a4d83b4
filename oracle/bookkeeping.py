"""CPU oracle of the speculative-step bookkeeping (tests only).

TEST INFRASTRUCTURE: imported by tests/ only.

A host restatement with the reference's own data structures (Python lists and
a deque) of:
  * BlockManager.allocate / deallocate, mini_vllm/engine/block_manager.py:
    35-92 (prefix hashing with xxhash64 as in :36-41);
  * the spec block of LLMEngine.step, mini_vllm/engine/llm_engine.py:
    pre-allocation :111-128, apply :146-164, trim :170-181 and the rehash of
    the remaining blocks :182-194 (xxhash64, the reference's own dependency);
  * the verify staging of run_verify, model_runner.py:339-362;
  * the dirty-slot range of cleanup_rejected_kv_slots, model_runner.py:445-464.
"""
from __future__ import annotations

from collections import deque

import numpy as np
import xxhash


class Block:
    def __init__(self, block_id):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1
        self.token_ids = []

    def reset(self):
        self.ref_count = 1
        self.hash = -1
        self.token_ids = []


class Seq:
    def __init__(self, token_ids, max_tokens=64, ignore_eos=False):
        self.token_ids = list(token_ids)
        self.num_prompt_tokens = len(token_ids)
        self.max_tokens = max_tokens
        self.ignore_eos = ignore_eos
        self.block_table = []
        self.finished = False
        self.num_cached_tokens = 0

    def __len__(self):
        return len(self.token_ids)

    @property
    def last_token(self):
        return self.token_ids[-1]

    @property
    def num_completion_tokens(self):
        return len(self.token_ids) - self.num_prompt_tokens

    def block(self, i, bs):
        return self.token_ids[i * bs:(i + 1) * bs]


class BookState:
    def __init__(self, num_blocks, block_size, eos=-1):
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.free = deque(range(num_blocks))
        self.used = set()
        self.hash_to_block_id = {}
        self.eos = eos

    @staticmethod
    def compute_hash(token_ids, prefix=-1):
        h = xxhash.xxh64()
        if prefix != -1:
            h.update(prefix.to_bytes(8, "little"))
        h.update(np.array(token_ids).tobytes())
        return h.intdigest()

    # block_manager.py:43-54
    def _allocate_block(self, block_id):
        block = self.blocks[block_id]
        assert block.ref_count == 0
        block.reset()
        self.free.remove(block_id)
        self.used.add(block_id)
        return block

    def _deallocate_block(self, block_id):
        assert self.blocks[block_id].ref_count == 0
        self.used.remove(block_id)
        self.free.append(block_id)

    # block_manager.py:59-82
    def allocate(self, seq: Seq):
        assert not seq.block_table
        bs = self.block_size
        h = -1
        cache_miss = False
        nblocks = (len(seq) + bs - 1) // bs
        for i in range(nblocks):
            token_ids = seq.block(i, bs)
            h = self.compute_hash(token_ids, h) if len(token_ids) == bs else -1
            block_id = self.hash_to_block_id.get(h, -1)
            if block_id == -1 or self.blocks[block_id].token_ids != token_ids:
                cache_miss = True
            if cache_miss:
                block_id = self.free[0]
                block = self._allocate_block(block_id)
            else:
                seq.num_cached_tokens += bs
                if block_id in self.used:
                    block = self.blocks[block_id]
                    block.ref_count += 1
                else:
                    block = self._allocate_block(block_id)
            if h != -1:
                block.hash = h
                block.token_ids = token_ids
                self.hash_to_block_id[h] = block_id
            seq.block_table.append(block_id)

    # block_manager.py:84-92
    def deallocate(self, seq: Seq):
        for block_id in reversed(seq.block_table):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._deallocate_block(block_id)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    # llm_engine.py:111-128
    def prealloc(self, seqs, gamma):
        eligible = []
        for seq in seqs:
            if seq.finished:
                eligible.append(0)
                continue
            needed_blocks = (len(seq) + gamma + 1 + self.block_size - 1) // self.block_size
            blocks_needed = needed_blocks - len(seq.block_table)
            if blocks_needed > 0 and len(self.free) < blocks_needed:
                eligible.append(0)
                continue
            for _ in range(blocks_needed):
                block_id = self.free[0]
                block = self.blocks[block_id]
                block.reset()
                self.free.remove(block_id)
                self.used.add(block_id)
                seq.block_table.append(block_id)
            eligible.append(1)
        return eligible

    # model_runner.py:339-362
    def prepare(self, seqs, draft_tokens):
        ids, pos, slots, cu_q, cu_k = [], [], [], [0], [0]
        for i, seq in enumerate(seqs):
            verify_tokens = [seq.last_token] + list(draft_tokens[i])
            start_pos = len(seq) - 1
            for j, tok in enumerate(verify_tokens):
                p = start_pos + j
                ids.append(tok)
                pos.append(p)
                bi = p // self.block_size
                if bi >= len(seq.block_table):
                    slots.append(-1)
                else:
                    slots.append(seq.block_table[bi] * self.block_size + p % self.block_size)
            cu_q.append(cu_q[-1] + len(verify_tokens))
            cu_k.append(cu_k[-1] + start_pos + len(verify_tokens))
        return ids, pos, slots, cu_q, cu_k

    # model_runner.py:445-464 (dirty_mode 0) or the exact range (dirty_mode 1)
    def dirty_slots(self, seq, accepted_len, gamma, dirty_mode):
        cur_len = len(seq)
        old_len = cur_len - accepted_len
        if dirty_mode == 0:
            lo, hi = old_len + accepted_len, old_len + gamma + 1
        else:
            lo, hi = cur_len - 1, old_len + gamma
        out = []
        for p in range(lo, hi):
            if p < 0:
                continue
            bi = p // self.block_size
            if bi < len(seq.block_table):
                out.append(seq.block_table[bi] * self.block_size + p % self.block_size)
        return out

    # llm_engine.py:146-181
    def commit(self, seqs, accepted_lists, gamma, dirty_mode=None):
        appended = []
        dirty = []
        for seq, accepted in zip(seqs, accepted_lists):
            n = 0
            if not seq.finished:
                for tok in accepted:
                    seq.token_ids.append(tok)
                    n += 1
                    if (not seq.ignore_eos and tok == self.eos) or \
                            seq.num_completion_tokens == seq.max_tokens:
                        seq.finished = True
                        self.deallocate(seq)
                        break
            appended.append(n)
            if dirty_mode is not None:
                if seq.finished or n == 0:
                    dirty.append([])
                else:
                    dirty.append(self.dirty_slots(seq, n, gamma, dirty_mode))
        for seq in seqs:
            if not seq.finished:
                needed_blocks = (len(seq) + self.block_size - 1) // self.block_size
                while len(seq.block_table) > needed_blocks:
                    block_id = seq.block_table.pop()
                    block = self.blocks[block_id]
                    block.ref_count -= 1
                    if block.ref_count == 0:
                        self.used.discard(block_id)
                        self.free.append(block_id)
                self.rehash(seq)
        return appended, dirty

    # llm_engine.py:182-194: full blocks without a hash get one (the previous
    # block's hash as prefix), a partial last block loses its hash
    def rehash(self, seq):
        bs = self.block_size
        for bi, block_id in enumerate(seq.block_table):
            block = self.blocks[block_id]
            is_last = bi == len(seq.block_table) - 1
            full = (not is_last) or (len(seq) % bs == 0)
            if full and block.hash == -1:
                token_ids = seq.block(bi, bs)
                prefix = self.blocks[seq.block_table[bi - 1]].hash if bi > 0 else -1
                h = self.compute_hash(token_ids, prefix)
                block.hash = h
                block.token_ids = token_ids
                self.hash_to_block_id[h] = block_id
            elif not full and block.hash != -1:
                block.hash = -1
                block.token_ids = []

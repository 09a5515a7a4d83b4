"""GPU parity of the spec-step bookkeeping kernels.

Random multi-step runs drive the oracle (oracle/bookkeeping.py, the
reference's own data structures) and the device state through the same
pre-allocation, staging and commit steps; after every step the whole device
state must equal the oracle's: lengths, token histories, block tables, free
deque contents in order, reference counts, finished flags, staging outputs,
dirty slots and block hashes (bit-exact integers).
"""
import numpy as np
import pytest
import torch

from oracle.bookkeeping import BookState, Seq

pytestmark = pytest.mark.gpu


def to_device(hv, bm, seqs, W, T, dev):
    B = len(seqs)
    st = hv.ops.SpecStateTensors(B, W, T, len(bm.blocks), bm.block_size, bm.eos, dev)
    lens = [len(s) for s in seqs]
    st.context_lens.copy_(torch.tensor(lens, dtype=torch.int32))
    st.num_prompt.copy_(torch.tensor([s.num_prompt_tokens for s in seqs], dtype=torch.int32))
    st.max_tokens.copy_(torch.tensor([s.max_tokens for s in seqs], dtype=torch.int32))
    st.ignore_eos.copy_(torch.tensor([int(s.ignore_eos) for s in seqs], dtype=torch.int32))
    st.finished.copy_(torch.tensor([int(s.finished) for s in seqs], dtype=torch.int32))
    bt = np.full((B, W), -1, np.int32)
    tok = np.zeros((B, T), np.int64)
    for i, s in enumerate(seqs):
        bt[i, :len(s.block_table)] = s.block_table
        tok[i, :len(s)] = s.token_ids
    st.block_tables.copy_(torch.from_numpy(bt))
    st.num_seq_blocks.copy_(torch.tensor([len(s.block_table) for s in seqs], dtype=torch.int32))
    st.tokens.copy_(torch.from_numpy(tok))
    N = len(bm.blocks)
    ring = np.zeros(N, np.int32)
    ring[:len(bm.free)] = list(bm.free)
    st.free_ring.copy_(torch.from_numpy(ring))
    st.free_hdr.copy_(torch.tensor([0, len(bm.free)], dtype=torch.int32))
    st.ref_count.copy_(torch.tensor([b.ref_count for b in bm.blocks], dtype=torch.int32))
    st.block_hash.copy_(torch.tensor([as_i64(b.hash) for b in bm.blocks], dtype=torch.int64))
    return st


def as_i64(h):
    """A block hash (xxh64 digest, or -1) as the device's int64."""
    return h - (1 << 64) if h >= (1 << 63) else h


def assert_same_state(st, bm, seqs):
    torch.cuda.synchronize()
    B = len(seqs)
    lens = st.context_lens.cpu().numpy()
    assert lens.tolist() == [len(s) for s in seqs]
    assert st.finished.cpu().tolist() == [int(s.finished) for s in seqs]
    nb = st.num_seq_blocks.cpu().numpy()
    bt = st.block_tables.cpu().numpy()
    tok = st.tokens.cpu().numpy()
    for i, s in enumerate(seqs):
        assert nb[i] == len(s.block_table), (i, nb[i], s.block_table)
        assert bt[i, :nb[i]].tolist() == s.block_table
        assert (bt[i, nb[i]:] == -1).all()
        assert tok[i, :len(s)].tolist() == s.token_ids
    hdr = st.free_hdr.cpu().tolist()
    ring = st.free_ring.cpu().numpy()
    N = len(bm.blocks)
    free = [int(ring[(hdr[0] + k) % N]) for k in range(hdr[1])]
    assert free == list(bm.free)
    refs = st.ref_count.cpu().numpy()
    used = sorted({b for s in seqs for b in s.block_table})
    for b in used:
        assert refs[b] == bm.blocks[b].ref_count, (b, refs[b], bm.blocks[b].ref_count)
    # every block's hash (xxh64 by the xxhash library in the oracle), free ones included
    hashes = st.block_hash.cpu().tolist()
    assert hashes == [as_i64(b.hash) for b in bm.blocks]


@pytest.mark.parametrize("seed", range(6))
def test_random_spec_steps_match_oracle(hv, cuda, seed):
    rng = np.random.default_rng(100 + seed)
    bs = int(rng.choice([4, 16, 256]))
    B = int(rng.integers(1, 40))
    num_blocks = int(rng.integers(B * 2, B * 6 + 8)) if bs < 256 else B * 3 + 4
    W, T = 64, 4096
    eos = 5
    bm = BookState(num_blocks, bs, eos=eos)
    shared = list(rng.integers(0, 9, size=bs))  # common prefix -> shared blocks
    seqs = []
    for i in range(B):
        plen = int(rng.integers(1, 3 * bs))
        prompt = (shared + list(rng.integers(6, 9, size=plen)))[:max(plen, 1)] \
            if i % 3 == 0 else list(rng.integers(6, 9, size=plen))
        s = Seq(prompt, max_tokens=int(rng.integers(2, 30)), ignore_eos=bool(i % 4 == 1))
        if len(bm.free) >= (len(s) + bs - 1) // bs + 1:
            bm.allocate(s)
            seqs.append(s)
    if not seqs:
        pytest.skip("no sequence fits")
    st = to_device(hv, bm, seqs, W, T, cuda)
    assert_same_state(st, bm, seqs)
    print(f"seed={seed} bs={bs} B={len(seqs)} blocks={num_blocks}", flush=True)
    for step in range(12):
        gamma = int(rng.integers(1, 8))
        # pre-allocation over the whole batch
        elig_ref = bm.prealloc(seqs, gamma)
        elig = hv.ops.spec_prealloc(st, gamma)
        assert elig.cpu().tolist() == elig_ref, (step, elig.cpu().tolist(), elig_ref)
        assert_same_state(st, bm, seqs)
        # staging and commit for the eligible sequences (device runs the full
        # batch; ineligible rows offer no tokens)
        drafts = rng.integers(0, 9, size=(len(seqs), gamma)).astype(np.int64)
        ids, pos, slots, cq, ck = hv.ops.verify_prepare(st, torch.from_numpy(drafts).to(cuda),
                                                        gamma)
        r_ids, r_pos, r_slots, r_cq, r_ck = bm.prepare(seqs, drafts)
        torch.cuda.synchronize()
        live = [i for i, s in enumerate(seqs) if not s.finished]
        R = gamma + 1
        for i in live:
            assert ids.cpu().numpy()[i * R:(i + 1) * R].tolist() == r_ids[i * R:(i + 1) * R]
            assert pos.cpu().numpy()[i * R:(i + 1) * R].tolist() == r_pos[i * R:(i + 1) * R]
            assert slots.cpu().numpy()[i * R:(i + 1) * R].tolist() == r_slots[i * R:(i + 1) * R]
        assert cq.cpu().tolist() == r_cq and ck.cpu().tolist() == r_ck
        out = np.full((len(seqs), R), -1, np.int64)
        olen = np.zeros(len(seqs), np.int32)
        acc = []
        for i, s in enumerate(seqs):
            # ineligible rows offer tokens too: the commit must skip them by `eligible`
            n = int(rng.integers(1, R + 1)) if elig_ref[i] else int(rng.integers(0, R + 1))
            toks = list(rng.integers(0, 9, size=n))
            out[i, :n] = toks
            olen[i] = n
            acc.append(toks)
        batch = [s for s, e in zip(seqs, elig_ref) if e]
        batch_acc = [a for a, e in zip(acc, elig_ref) if e]
        mode = step % 2
        app_ref, dirty_ref = bm.commit(batch, batch_acc, gamma, dirty_mode=mode)
        app, dirty = hv.ops.spec_commit(st, gamma, torch.from_numpy(out).to(cuda),
                                        torch.from_numpy(olen).to(cuda), dirty_mode=mode,
                                        eligible=elig)
        torch.cuda.synchronize()
        app_c = app.cpu().numpy()
        dirty_c = dirty.cpu().numpy()
        k = 0
        for i, e in enumerate(elig_ref):
            if e:
                assert app_c[i] == app_ref[k]
                d = dirty_c[i][dirty_c[i] >= 0].tolist()
                assert d == dirty_ref[k], (step, i, d, dirty_ref[k])
                k += 1
            else:
                assert app_c[i] == 0
        assert_same_state(st, bm, seqs)


def test_zero_kv_slots(hv, cuda):
    L, nb, bs, H, D = 3, 4, 16, 2, 128
    cache = torch.randn((2, L, nb, bs, H, D), device=cuda).to(torch.bfloat16)
    ref = cache.clone()
    slots = torch.tensor([5, -1, 17, 63], dtype=torch.int32, device=cuda)
    hv.ops.zero_kv_slots(cache, slots)
    flat = ref.view(2, L, nb * bs, H, D)
    for s in [5, 17, 63]:
        flat[:, :, s] = 0
    torch.cuda.synchronize()
    assert torch.equal(cache, ref)

"""The speculative step on one MI355X: K draft blocks denoised by the draft,
verified by the target in one cached forward, greedy acceptance.

Mirrors the reference's K-block loop (speculative_decoding/speculative_decode.py:
840-953 with the greedy match of mrs.py:111-146, the fused denoise graphs of
cache_aware.py:840-1075 and the multi-block verify of verify.py:421-700),
with the target's verify run against its KV cache: its rows are only the K
draft blocks (data, mask), not the whole prompt.  Per iteration:

  draft   K block graphs; each folds the previous block in as a committed
          prefix (its K/V rewritten in place by the first of ds denoise
          forwards, [prefix 4 | block 4] rows; the rest run the block's 4
          rows), each unmasking ceil(remaining / steps left) positions by
          confidence (denoise_select)
  verify  one target forward of [the blocks the last acceptance committed |
          K x (4 data + 4 mask)] rows: the committed blocks are folded in
          ahead of the verify rows and write their K/V to their permanent
          slots (block-causal among themselves, seen by every verify row), so
          no separate extend forward streams the target's weights again; the
          lm_head runs on the mask rows only, whose argmax is all the
          acceptance reads (softmax_argmax)
  accept  greedy match per block with first-reject truncation; a rejected
          block is committed padded with the draft's own tokens
          (partial_block_fill = "draft_argmax")

``fold=False`` keeps the reference's separate extend (cache_aware.py:
1202-1259, _extend_cache_graph): one target forward of the committed
block(s) storing their K/V, on a second HIP stream where it overlaps the next
iteration's draft blocks (which only need the committed ids; the next verify
waits for it), or in line with ``overlap=False``.  Every mode commits the
same tokens.

``pipelined=True`` adds the reference's optimistic execution
(cache_aware.py:2169-2668, speculative_generate_with_kv_cache_pipelined, there
across two GPUs with K = 1; here on two streams of one GPU, any K): while the
target verifies iteration N on the main stream, the draft already denoises
iteration N + 1's blocks on a side stream as if every block of N were
accepted.  On full acceptance those drafts are used as they are; otherwise
they are dropped (rollback: the context is what acceptance committed, and the
slots the optimistic drafts wrote past it are rewritten or masked out) and the
blocks are drafted again.  Both modes commit exactly the same tokens.

The committed context lives in permanent cache slots [0, ctx); a forward's
rows write their K/V at slots ctx.. in row order (past the committed context,
so a later forward overwrites them), and each row's mask comes from
block_mask on the device.  Every forward is a captured HIP graph whose
per-iteration inputs (ids, positions, slots, mask, valid length) are device
buffers refreshed before the replay.  A forward has one graph per bound on
the attention's valid length: the one-launch attention's limit while the
context fits it, the whole cache beyond (the device-side valid length then
lowers the bound at run time).  One host synchronisation per iteration reads
the 2 x K x 4 ids the acceptance needs.
"""
from __future__ import annotations

import torch

from kernels.attention_fused import ONE_LAUNCH_SLOTS, block_mask
from kernels.logits_fused import denoise_select, softmax_argmax

from .model import SynthModel
from .verify import MASK_TOKEN_ID, accept_blocks


def unmask_schedule(n_masks: int, steps: int):
    """Positions unmasked per denoise step (cache_aware.py:869-877)."""
    out, rem = [], n_masks
    for s in range(steps):
        n = -(-rem // (steps - s))
        if n <= 0:
            break
        out.append(n)
        rem -= n
    return out


# attention bounds, one captured graph each, up to the one-launch form's
# limit (the chunked form sizes its chunks for the bound; the device-side
# length trims the work of either form)
GRAPH_BOUNDS = (1024, 2048, ONE_LAUNCH_SLOTS)


def valid_bound(cache_len: int, end: int) -> int:
    """Host-side bound on the attention's valid length for a forward whose
    rows end at slot ``end``: the first of ``GRAPH_BOUNDS`` that holds it
    (below the cache's length), otherwise the whole cache."""
    for bound in GRAPH_BOUNDS:
        if end <= bound < cache_len:
            return bound
    return cache_len


class _Graphed:
    """A forward captured over static device buffers, one graph per key (the
    attention's valid-length bound).  ``head_rows``: the rows whose logits
    the forward computes (all when None)."""

    def __init__(self, rows: int, n_cols: int, device, head_rows: torch.Tensor | None = None):
        self.head_rows = head_rows
        self.ids = torch.zeros(rows, dtype=torch.int64, device=device)
        self.pos = torch.zeros(rows, dtype=torch.int64, device=device)
        self.slots = torch.zeros(rows, dtype=torch.int64, device=device)
        self.mask = torch.zeros(rows, (n_cols + 3) // 4 * 4, dtype=torch.bool, device=device)
        self.valid = torch.zeros(1, dtype=torch.int64, device=device)
        self.graphs, self.outs = {}, {}

    def set_span(self, start: int, ctx_len: int, rows: int):
        """Rows at positions/slots start.. (row order); valid = start + rows."""
        ar = torch.arange(start, start + rows, dtype=torch.int64, device=self.pos.device)
        self.pos.copy_(ar)
        self.slots.copy_(ar)
        self.valid.fill_(start + rows)

    def replay(self, key, body):
        """Replay the graph of ``key``, capturing ``body`` first if needed."""
        if key not in self.graphs:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                body()                               # warm: allocations, lazy init
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.outs[key] = body()
            self.graphs[key] = graph
        self.graphs[key].replay()
        return self.outs[key]


class SpecRunner:
    """Greedy speculative decoding of one sequence with a draft and a target
    resident on one GPU."""

    def __init__(self, draft: SynthModel, target: SynthModel, block_length: int = 4, denoise_steps: int = 4,
                 k_blocks: int = 4, mask_token_id: int = MASK_TOKEN_ID, overlap: bool = True,
                 pipelined: bool = False, fold: bool = True):
        self.draft, self.target = draft, target
        self.bl, self.ds, self.K = block_length, denoise_steps, k_blocks
        self.mask_id = mask_token_id
        self.dev = draft.device
        self.schedule = unmask_schedule(block_length, denoise_steps)
        bl, K = block_length, k_blocks
        dcols, tcols = draft.cache.full_len, target.cache.full_len
        self._dg = _Graphed(2 * bl, dcols, self.dev)                  # [prefix | block]
        self._vg = {}          # folded committed blocks c -> [c blocks | K x (data, mask)] graph
        self._eg = {}                                                 # committed blocks -> extend graph
        self._step_map = torch.full((bl,), -1, dtype=torch.int64, device=self.dev)
        self.draft_blocks = torch.zeros(K, bl, dtype=torch.int64, device=self.dev)
        self.step_maps = torch.zeros(K, bl, dtype=torch.int64, device=self.dev)
        self.overlap = overlap
        self.pipelined = pipelined
        self.fold = fold
        self._pending = []        # committed blocks not yet in the target cache (folded into the next verify)
        self._verify_graph_now = None
        self.side = torch.cuda.Stream(device=self.dev)      # default priority
        self.draft_stream = torch.cuda.Stream(device=self.dev)
        self._extend_done = None
        self._verify_ready = None
        self._verify_logits = {}      # (folded blocks, bound) -> the verify graph's logits output
        self._verify_key = None
        self._draft_done = None       # optimistic drafts still running on draft_stream
        self._have_next = False       # draft_blocks hold valid drafts for the next iteration
        self.stats = {"optimistic_used": 0, "optimistic_dropped": 0}
        self.ctx = 0
        self.tokens = []          # generated tokens (accepted + bonus)
        self.history = []         # the committed context: prompt + committed blocks

    # ----------------------------------------------------------- prefill
    @torch.inference_mode()
    def prefill(self, prompt_ids: torch.Tensor):
        """Both caches take the prompt (block-causal over blocks of
        block_length, as the SDAR prompt rule; not part of the timed step)."""
        n = int(prompt_ids.numel())
        if n % self.bl:
            raise ValueError("prompt length must be a multiple of the block length")
        if n > min(self.draft.cache.full_len, self.target.cache.full_len):
            raise ValueError("prompt longer than the KV caches")
        ids = prompt_ids.to(self.dev, torch.int64)
        ar = torch.arange(n, device=self.dev)
        blk = ar // self.bl
        for m in (self.draft, self.target):
            mask = torch.zeros(n, m.cache.full_len, dtype=torch.bool, device=self.dev)
            mask[:, :n] = blk[None, :] <= blk[:, None]
            m.forward(ids, ar, ar, mask, valid_len=n, head=False)
        self.ctx = n
        self.history = prompt_ids.tolist()
        self.last_block = ids[n - self.bl:].clone()
        torch.cuda.synchronize()

    # ------------------------------------------------------------ graphs
    def _draft_body(self, bound):
        """ds denoise forwards of one block.  The first carries the prefix
        rows, which writes their K/V; the later ones run the block's rows
        alone, reading the prefix from the cache (the reference re-encodes the
        prefix in every step, cache_aware.py:851-861, which is idempotent)."""
        g, bl = self._dg, self.bl
        g.ids[bl:].fill_(self.mask_id)
        self._step_map.fill_(-1)
        for step, n_u in enumerate(self.schedule):
            # the rows sit at the last slots of the valid range (set_span)
            if step == 0:
                logits = self.draft.forward(g.ids, g.pos, g.slots, g.mask, valid_len=bound,
                                            valid_len_dev=g.valid, head_rows=slice(bl, 2 * bl), rows_at_end=True)
            else:
                logits = self.draft.forward(g.ids[bl:], g.pos[bl:], g.slots[bl:], g.mask[bl:],
                                            valid_len=bound, valid_len_dev=g.valid, rows_at_end=True)
            denoise_select(logits, g.ids[bl:], self.mask_id, n_u, step, self._step_map)
        return None

    def _verify_graph(self, c: int) -> _Graphed:
        """The verify graph with ``c`` committed blocks folded in: rows
        [c blocks | K x (bl data, bl mask)], logits of the mask rows only."""
        g = self._vg.get(c)
        if g is None:
            bl, K = self.bl, self.K
            n0 = c * bl
            mask_rows = [n0 + 2 * k * bl + bl + j for k in range(K) for j in range(bl)]
            g = _Graphed(n0 + 2 * K * bl, self.target.cache.full_len, self.dev,
                         head_rows=torch.tensor(mask_rows, dtype=torch.int64, device=self.dev))
            self._vg[c] = g
        return g

    def _verify_body(self, g, key):
        logits = self.target.forward(g.ids, g.pos, g.slots, g.mask, valid_len=key[1], valid_len_dev=g.valid,
                                     head_rows=g.head_rows, rows_at_end=True)
        self._verify_logits[key] = logits
        ids, _ = softmax_argmax(logits)
        return ids

    def _extend_body(self, g, bound):
        self.target.forward(g.ids, g.pos, g.slots, g.mask, valid_len=bound, valid_len_dev=g.valid, head=False,
                            rows_at_end=True)
        return None

    def _extend_graph(self, n_blocks: int):
        g = self._eg.get(n_blocks)
        if g is None:
            g = _Graphed(n_blocks * self.bl, self.target.cache.full_len, self.dev)
            self._eg[n_blocks] = g
        return g

    def history_ids(self):
        return list(self.history)

    # ---------------------------------------------------------- one step
    @torch.inference_mode()
    def draft_blocks_(self, ctx: int | None = None, last_block: torch.Tensor | None = None):
        """K blocks; block k folds block k - 1 (the last committed block for
        k = 0) in as its prefix.  ``ctx`` / ``last_block`` default to the
        committed state (the optimistic drafts pass the assumed one)."""
        g, bl, dcols = self._dg, self.bl, self.draft.cache.full_len
        ctx = self.ctx if ctx is None else ctx
        last_block = self.last_block if last_block is None else last_block
        for k in range(self.K):
            start = ctx - bl + k * bl                 # prefix position
            g.ids[:bl].copy_(last_block if k == 0 else self.draft_blocks[k - 1])
            g.set_span(start, start, 2 * bl)
            block_mask(dcols, start, start, n_prefix=bl, n_free=bl, out=g.mask)
            bound = valid_bound(dcols, start + 2 * bl)
            g.replay(bound, lambda: self._draft_body(bound))
            self.draft_blocks[k].copy_(g.ids[bl:])
            self.step_maps[k].copy_(self._step_map)

    @torch.inference_mode()
    def verify_(self):
        if self._extend_done is not None:            # the target cache must hold the last commit
            torch.cuda.current_stream().wait_event(self._extend_done)
            self._extend_done = None
        bl, K = self.bl, self.K
        c = len(self._pending)
        g = self._verify_graph(c)
        n0 = c * bl
        p0 = self.ctx - n0                           # the folded blocks' permanent slots [p0, ctx)
        if c:
            folded = torch.tensor([t for b in self._pending for t in b], dtype=torch.int64)
            g.ids[:n0].copy_(folded.to(self.dev, non_blocking=True))
        ids = g.ids[n0:].view(K, 2, bl)
        ids[:, 0].copy_(self.draft_blocks)
        ids[:, 1].fill_(self.mask_id)
        ar = torch.arange(p0, self.ctx + 2 * K * bl, dtype=torch.int64, device=self.dev)
        g.slots.copy_(ar)                            # folded blocks, then the verify rows' scratch
        g.pos[:n0].copy_(ar[:n0])
        pos = torch.arange(self.ctx, self.ctx + K * bl, dtype=torch.int64, device=self.dev).view(K, 1, bl)
        g.pos[n0:].view(K, 2, bl).copy_(pos.expand(K, 2, bl))   # masks share the data positions
        g.valid.fill_(self.ctx + 2 * K * bl)
        block_mask(self.target.cache.full_len, p0, p0, n_prefix=n0, step_maps=self.step_maps,
                   block_length=bl, block_size=self.ds, out=g.mask)
        bound = valid_bound(self.target.cache.full_len, self.ctx + 2 * K * bl)
        # the verify's inputs are set: later work may overwrite draft_blocks / step_maps
        self._verify_ready = torch.cuda.Event()
        self._verify_ready.record()
        self._verify_key = (c, bound)
        self._verify_graph_now = g
        out = g.replay(bound, lambda: self._verify_body(g, (c, bound)))
        self._pending = []                           # their K/V are in the target cache now
        return out.view(K, bl)

    @property
    def last_verify_logits(self) -> torch.Tensor:
        """Logits [K * bl, V] of the last verify's mask rows (block k's mask
        rows at k * bl ..), valid until the same graph replays again."""
        return self._verify_logits[self._verify_key]

    @property
    def last_verify_ids(self) -> torch.Tensor:
        """The last verify's argmax ids at the mask rows, [K, bl]."""
        g = self._verify_graph_now
        return g.outs[self._verify_key[1]].view(self.K, self.bl)

    @property
    def last_verify_drafts(self) -> torch.Tensor:
        """The drafts the last verify checked, [K, bl] (a view of its inputs)."""
        g = self._verify_graph_now
        return g.ids[self._verify_key[0] * self.bl:].view(self.K, 2, self.bl)[:, 0]

    @property
    def last_verify_graph(self) -> _Graphed:
        return self._verify_graph_now

    @torch.inference_mode()
    def extend_(self, blocks, start: int | None = None):
        """The committed ``blocks`` through the target, storing their K/V at
        slots ``start`` .. (default: the committed context's end)."""
        n = len(blocks)
        start = self.ctx if start is None else start
        g = self._extend_graph(n)
        ids = torch.tensor([t for b in blocks for t in b], dtype=torch.int64)
        main = torch.cuda.current_stream()
        stream = self.side if self.overlap else main
        if self.overlap:
            stream.wait_stream(main)                  # after the verify that wrote its rows
        with torch.cuda.stream(stream):
            g.ids.copy_(ids.to(self.dev, non_blocking=True))
            g.set_span(start, start, n * self.bl)
            block_mask(self.target.cache.full_len, start, start, n_prefix=n * self.bl, block_length=self.bl,
                       out=g.mask)
            bound = valid_bound(self.target.cache.full_len, start + n * self.bl)
            g.replay(bound, lambda: self._extend_body(g, bound))
            if self.overlap:
                self._extend_done = torch.cuda.Event()
                self._extend_done.record(stream)

    @torch.inference_mode()
    def flush(self):
        """Write the committed blocks still waiting to be folded into a verify
        into the target cache now (an extend), so that it holds the whole
        committed context."""
        if self._pending:
            n = len(self._pending)
            self.extend_(self._pending, start=self.ctx - n * self.bl)
            self._pending = []

    def finish(self):
        """Wait for work still running on the side streams (an extend, an
        optimistic draft)."""
        if self._extend_done is not None:
            torch.cuda.current_stream().wait_event(self._extend_done)
            self._extend_done = None
        if self._draft_done is not None:
            torch.cuda.current_stream().wait_event(self._draft_done)
            self._draft_done = None

    @torch.inference_mode()
    def step(self, events=None):
        """One iteration -> (generated tokens, accepted draft tokens).  With
        ``events`` (four torch.cuda.Event), their records bracket the draft,
        verify, acceptance and extend phases on the current stream."""
        # the verify's scratch rows (and the optimistic drafts') reach
        # ctx + 2 K bl slots; past the caches the step would write nowhere
        cap = min(self.draft.cache.full_len, self.target.cache.full_len)
        if self.ctx + 2 * self.K * self.bl > cap:
            raise RuntimeError(f"speculative step: context {self.ctx} + {2 * self.K * self.bl} scratch rows "
                               f"exceeds the KV caches' {cap} slots")
        main = torch.cuda.current_stream()
        if events:
            events[0].record()
        if self._draft_done is not None:              # optimistic drafts finish before use or redo
            main.wait_event(self._draft_done)
            self._draft_done = None
        if self._pending and not self.fold:           # switched out of the folding mode
            self.flush()
        if not self._have_next:
            self.draft_blocks_()
        self._have_next = False
        if events:
            events[1].record()
        target_ids = self.verify_()
        if self.pipelined:
            # iteration N + 1's drafts, assuming every block of N is accepted,
            # on their own stream while the verify runs
            K, bl = self.K, self.bl
            with torch.cuda.stream(self.draft_stream):
                self.draft_stream.wait_event(self._verify_ready)
                self.draft_blocks_(ctx=self.ctx + K * bl, last_block=self.last_verify_drafts[K - 1])
                self._draft_done = torch.cuda.Event()
                self._draft_done.record(self.draft_stream)
        if events:
            events[2].record()
        drafted = self.last_verify_drafts                              # the drafts this verify checked
        both = torch.stack([drafted, target_ids]).cpu()                # the one host sync
        committed, generated, n_acc = accept_blocks(both[0].tolist(), both[1].tolist(), self.bl)
        if self.pipelined:
            self._have_next = n_acc == self.K * self.bl
            self.stats["optimistic_used" if self._have_next else "optimistic_dropped"] += 1
        if events:
            events[3].record()
        if self.fold:
            self._pending = committed                 # rows of the next verify
        else:
            self.extend_(committed)
        self.ctx += self.bl * len(committed)
        self.history.extend(t for b in committed for t in b)
        self.last_block = torch.tensor(committed[-1], dtype=torch.int64, device=self.dev)
        self.tokens.extend(generated)
        return generated, n_acc

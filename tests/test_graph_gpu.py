"""ar_gpt_train_step_graph: the whole training step replayed from a HIP
graph gives the eager step's results bit for bit.  Several replays, each on
a new batch copied into the recorded buffers and at a different schedule
point (new step scalars), with eager work and synchronisations in between;
every replay is checked against an eager model stepped identically."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CONFIG1 = dict(sequence_len=64, vocab_size=512, n_layer=2, n_head=2, n_kv_head=2, n_embd=128, head_dim=64,
               kv_dim=128)
WIDE = dict(sequence_len=256, vocab_size=1024, n_layer=4, n_head=2, n_kv_head=2, n_embd=256, head_dim=128,
            kv_dim=256)


@pytest.mark.parametrize("cfg,B,T,precision,period", [(CONFIG1, 2, 64, 0, 0), (WIDE, 2, 256, 1, 256)])
def test_graph_replay_matches_eager(cfg, B, T, precision, period):
    import torch
    import gpu_util as gu
    from autoresearch_amd.model import GPT, GPTConfig
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        eager = GPT(GPTConfig(**cfg), B, T, precision=precision, rope_period=period)
        graph = GPT(GPTConfig(**cfg), B, T, precision=precision, rope_period=period)
        eager.init_weights(3)
        graph.init_weights(3)
        xin = torch.zeros(B * T, dtype=torch.int64, device="cuda")
        xtg = torch.zeros(B * T, dtype=torch.int64, device="cuda")
        r = np.random.default_rng(5)
        for step, progress in enumerate([0.0, 0.2, 0.55, 0.8, 0.95]):
            stream = r.integers(0, cfg["vocab_size"], (B, T + 1)).astype(np.int64)
            x = gu.dev(np.ascontiguousarray(stream[:, :-1]).ravel())
            y = gu.dev(np.ascontiguousarray(stream[:, 1:]).ravel())
            xin.copy_(x)
            xtg.copy_(y)
            le = eager.train_step(x, y, progress)
            lg = graph.train_step_graph(xin, xtg, progress)
            torch.cuda.synchronize()
            assert le == lg, (step, le, lg)
            np.testing.assert_array_equal(gu.host(graph.params()), gu.host(eager.params()), err_msg=f"step {step}")
            np.testing.assert_array_equal(gu.host(graph.token_loss()), gu.host(eager.token_loss()))
            _ = (x.float() * 2).sum().item()  # unrelated eager work between replays
        eager.close()
        graph.close()


def test_graph_needs_a_stream():
    import torch
    import gpu_util as gu
    from autoresearch_amd._lib import ArError
    from autoresearch_amd.model import GPT, GPTConfig
    with torch.cuda.stream(torch.cuda.default_stream()):
        m = GPT(GPTConfig(**CONFIG1), 2, 64, precision=0)
        x = gu.dev(np.zeros(128, np.int64))
        if torch.cuda.current_stream().cuda_stream == 0:
            with pytest.raises(ArError, match="null stream"):
                m.train_step_graph(x, x)
        m.close()

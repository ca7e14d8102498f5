/* A C client of libmitok: includes include/mitok.h as a foreign caller
 * would (the Rust -sys crate binds the same prototypes) and drives the
 * token loop through the C ABI only.
 *
 * Built by tests/test_abi.py with -Wall -Werror -std=c11 against the header;
 * a prototype that disagrees with a call here fails the build.  With a GPU
 * (./abi_client run) it builds a two-layer model from seeds, runs
 * mitok_generate, then mitok_prefill + mitok_decode_step for the same tokens,
 * and prints both id lists; the test compares them. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mitok.h"

#define CHECK(call)                                                          \
  do {                                                                       \
    int rc_ = (call);                                                        \
    if (rc_ != MITOK_OK) {                                                   \
      fprintf(stderr, "%s -> %d: %s\n", #call, rc_, mitok_last_error());     \
      return 1;                                                              \
    }                                                                        \
  } while (0)

enum { VOCAB = 97, DIM = 16, HEADS = 2, FFN = 32, CTX = 64, PROMPT = 7, NEW = 9 };

static int build(mitok_network* net) {
  CHECK(mitok_add_embedding(net, VOCAB, DIM, NULL));
  for (int l = 0; l < 2; ++l) {
    CHECK(mitok_add_norm(net, DIM, 1e-5, NULL, NULL));
    CHECK(mitok_add_self_attention(net, HEADS, DIM, CTX, 1e-12, NULL, NULL, NULL, NULL, NULL, NULL));
    CHECK(mitok_add_feed_forward(net, DIM, FFN, NULL, NULL, NULL, NULL));
  }
  CHECK(mitok_add_linear(net, DIM, VOCAB, NULL, NULL));
  CHECK(mitok_add_softmax(net, MITOK_PRODUCTION));
  CHECK(mitok_init_seeded(net, 42));
  return 0;
}

int main(int argc, char** argv) {
  if (argc < 2 || strcmp(argv[1], "run") != 0) {
    printf("abi_client: version %d\n", mitok_version());
    return 0;
  }
  int ndev = 0;
  CHECK(mitok_device_count(&ndev));
  if (ndev < 1) {
    fprintf(stderr, "no device\n");
    return 1;
  }
  mitok_network* net = NULL;
  CHECK(mitok_network_create(0, &net));
  if (build(net)) return 1;
  const uint32_t prompt[PROMPT] = {5, 17, 3, 60, 2, 44, 9};
  const uint32_t lens[1] = {PROMPT};
  uint32_t gen[NEW], step[NEW];
  CHECK(mitok_set_decode_plan(net, 1));
  CHECK(mitok_generate(net, prompt, lens, 1, PROMPT, NEW, gen, NULL));
  CHECK(mitok_prefill(net, prompt, lens, 1, PROMPT, &step[0], NULL));
  for (int t = 1; t < NEW; ++t) CHECK(mitok_decode_step(net, NULL, 1, &step[t], NULL));
  printf("generate:");
  for (int t = 0; t < NEW; ++t) printf(" %u", gen[t]);
  printf("\nsteps:");
  for (int t = 0; t < NEW; ++t) printf(" %u", step[t]);
  printf("\n");
  /* a decode step before prefill is a state error, not a crash */
  CHECK(mitok_reset(net));
  uint32_t one = 0;
  const int rc = mitok_decode_step(net, NULL, 1, &one, NULL);
  printf("decode_step after reset: %d\n", rc);
  mitok_network_destroy(net);
  return rc == MITOK_ERR_STATE ? 0 : 1;
}

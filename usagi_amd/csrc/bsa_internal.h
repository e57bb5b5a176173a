// Internal to libusagi_bsa.so: the error state shared by its translation units.
#ifndef USAGI_BSA_INTERNAL_H
#define USAGI_BSA_INTERNAL_H

// Records a formatted message for usagi_bsa_last_error() on the calling thread; returns code.
__attribute__((visibility("hidden"), format(printf, 2, 3))) int usagi_bsa_fail(int code,
                                                                               const char* fmt,
                                                                               ...);

// Empties the calling thread's message (every entry point starts with it).
__attribute__((visibility("hidden"))) void usagi_bsa_clear_error(void);

#endif  // USAGI_BSA_INTERNAL_H
